// Short causal convolution ahead of GDN (gfx950 / CDNA4, wave64).
//
// In a Qwen3-Next-style layer the q, k and v projections, concatenated
// channel-wise ("mixed_qkv", C = 2 HQ 128 + HV 128 channels), pass through a
// depthwise causal conv1d of kernel size W (4) and SiLU before they become
// the GDN operators' q, k, v; decode keeps each sequence's last inputs as a
// conv state.  The reference operators take q, k, v after this step; these
// kernels perform it and write the results straight into the GDN input
// layout (q [T, HQ, 128], k [T, HQ, 128], v [T, HV, 128]), so no split copy
// follows.
//
//   y[t, c] = act(bias[c] + sum_w weight[c, w] h[t - (W - 1) + w, c])
//
// with h the sequence's inputs preceded by its conv state (S >= W - 1 inputs,
// oldest first) or zeros.  Arithmetic in fp32, bf16 in and out.  Both kernels
// are HBM-bound streams: each lane owns 8 adjacent channels (one 16-byte
// load / store per token), a sliding window of the last W - 1 inputs stays in
// registers, and a workgroup of 256 lanes covers 2048 channels of one tile of
// tokens.

#include "gdn_common.h"
#include "../../include/gdn_hip.h"

namespace {

using namespace gdn;

constexpr int kConvThreads = 256;
constexpr int kConvTile = 64;        // tokens per lane in the prefill kernel
constexpr int kMaxConvWidth = 4;
constexpr int kMaxStateLen = 8;

// Destination of channels c0 .. c0 + 7 of token t: the q, k or v tensor, each
// [tokens, width] row-major (cq, ck multiples of 8).
struct QkvOut {
  uint16_t* q;
  uint16_t* k;
  uint16_t* v;
  int cq, ck, cv;
};

__device__ __forceinline__ uint16_t* out_at(const QkvOut& o, int t, int c0) {
  if (c0 < o.cq) return o.q + size_t(t) * o.cq + c0;
  c0 -= o.cq;
  if (c0 < o.ck) return o.k + size_t(t) * o.ck + c0;
  return o.v + size_t(t) * o.cv + (c0 - o.ck);
}

__device__ __forceinline__ void load8(const uint16_t* p, float (&f)[8]) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  unpack_bf16x2(w.x, f[0], f[1]);
  unpack_bf16x2(w.y, f[2], f[3]);
  unpack_bf16x2(w.z, f[4], f[5]);
  unpack_bf16x2(w.w, f[6], f[7]);
}

__device__ __forceinline__ void store8(uint16_t* p, const float (&f)[8]) {
  *reinterpret_cast<uint4*>(p) = uint4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                                       pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])};
}

template <typename CuT>
__device__ __forceinline__ int clamp_cu(const CuT* cu, int n, int T) {
  long long v = (long long)cu[n];
  return int(v < 0 ? 0 : (v > T ? T : v));
}

// The sequence holding token t: the largest n < N with cu[n] <= t (empty
// sequences before it are skipped), cu clamped into [0, T].
template <typename CuT>
__device__ int seq_of(const CuT* cu, int N, int T, int t) {
  int lo = 0, hi = N;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (clamp_cu(cu, mid, T) <= t) lo = mid;
    else hi = mid;
  }
  return lo;
}

template <bool kSilu>
__device__ __forceinline__ float activate(float y) {
  if constexpr (kSilu) return y * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-y * 1.44269504088896341f));
  else return y;
}

// Prefill: grid (ceil(C / 2048), ceil(T / 32) [+ 1 row for the states of
// empty sequences when st_out is given]).  st_out must not alias st_in: a
// sequence's start tile reads st_in while its end tile writes st_out.
template <int W, typename CuT, bool kSilu>
__global__ __launch_bounds__(kConvThreads) void gdn_qkv_conv1d_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ weight, const float* __restrict__ bias,
    const CuT* __restrict__ cu, int N, int T, int C, const uint16_t* __restrict__ st_in,
    uint16_t* __restrict__ st_out, int S, QkvOut o, int n_tiles) {
  const int c0 = 8 * (blockIdx.x * kConvThreads + threadIdx.x);
  if (c0 >= C) return;
  // value of channels c0.. of the input at token u for the sequence (n, bos):
  // x itself from bos on, before it the conv state (or zeros)
  auto hist_at = [&](int u, int n, int bos, float (&f)[8]) {
    if (u >= bos) {
      load8(x + size_t(u) * C + c0, f);
      return;
    }
    const int si = S - (bos - u);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      f[e] = (st_in != nullptr && si >= 0) ? bf16_bits_to_f32(st_in[(size_t(n) * C + c0 + e) * S + si]) : 0.f;
  };
  // the last S inputs of sequence n (ending at eos) -> st_out[n]
  auto write_state = [&](int n, int bos, int eos) {
    for (int si = 0; si < S; ++si) {
      float f[8];
      hist_at(eos - S + si, n, bos, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) st_out[(size_t(n) * C + c0 + e) * S + si] = f32_to_bf16_bits(f[e]);
    }
  };
  if (int(blockIdx.y) == n_tiles) {           // states of empty sequences: copies of their inputs
    for (int n = 0; n < N; ++n) {
      const int bos = clamp_cu(cu, n, T), eos = clamp_cu(cu, n + 1, T);
      if (eos <= bos) write_state(n, bos, bos);
    }
    return;
  }
  const int t0 = blockIdx.y * kConvTile;
  const int t1 = min(T, t0 + kConvTile);
  if (t0 >= t1) return;
  float wt[8][W], bs[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) wt[e][w] = weight[(c0 + e) * W + w];
    bs[e] = bias != nullptr ? bias[c0 + e] : 0.f;
  }
  // the tile in segments that lie in one sequence; within a segment the
  // inputs of eight tokens are loaded before their outputs are formed.
  // Tokens outside every sequence (before cu[0], at or past cu[N], or where
  // the ranges run backwards) get zero outputs; each pass of the loop
  // advances t, so the loop ends whatever cu holds.
  constexpr int kBatch = 8;
  auto zero_rows = [&](int u0, int u1) {
    const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int u = u0; u < u1; ++u) store8(out_at(o, u, c0), z);
  };
  for (int t = t0; t < t1;) {
    const int n = seq_of(cu, N, T, t);
    const int bos = clamp_cu(cu, n, T), eos = clamp_cu(cu, n + 1, T);
    if (t < bos) {                            // before the sequence's first token
      const int tb = min(t1, bos);
      zero_rows(t, tb);
      t = tb;
      continue;
    }
    const int te = min(t1, eos);
    if (te <= t) {                            // past the sequence's last token
      zero_rows(t, t1);
      break;
    }
    float hist[kMaxConvWidth - 1][8];         // hist[j]: input at token u - (W - 1) + j
#pragma unroll
    for (int j = 0; j < W - 1; ++j) hist_at(t - (W - 1) + j, n, bos, hist[j]);
    for (int u = t; u < te; u += kBatch) {
      uint4 raw[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        if (u + j < te) raw[j] = *reinterpret_cast<const uint4*>(x + size_t(u + j) * C + c0);
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (u + j >= te) break;
        float xs[8];
        unpack_bf16x2(raw[j].x, xs[0], xs[1]);
        unpack_bf16x2(raw[j].y, xs[2], xs[3]);
        unpack_bf16x2(raw[j].z, xs[4], xs[5]);
        unpack_bf16x2(raw[j].w, xs[6], xs[7]);
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = bs[e];
#pragma unroll
          for (int i = 0; i < W - 1; ++i) acc = fmaf(wt[e][i], hist[i][e], acc);
          acc = fmaf(wt[e][W - 1], xs[e], acc);
          y[e] = activate<kSilu>(acc);
        }
        store8(out_at(o, u + j, c0), y);
#pragma unroll
        for (int i = 0; i + 1 < W - 1; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) hist[i][e] = hist[i + 1][e];
#pragma unroll
        for (int e = 0; e < 8; ++e) hist[W - 2][e] = xs[e];
      }
    }
    if (st_out != nullptr && te == eos) write_state(n, bos, eos);
    t = te;
  }
}

// Decode: one token per sequence b, grid (ceil(C / 2048), ceil(B / kUpdSeqs)):
// a lane takes its 8 channels of kUpdSeqs sequences, so the channels' taps
// and bias are loaded once for all of them; every sequence's input and state
// words are issued before the first is used.  The state row state[slot]
// (slot = slot_ids[b], or b) is read, shifted by one with the token appended,
// and written back in place.  A slot outside [0, pool) leaves the state
// untouched and yields a zero output row.  The state length S is a
// compile-time W - 1 or W.
constexpr int kUpdSeqs = 8;

template <int W, int S, bool kSilu>
__global__ __launch_bounds__(kConvThreads) void gdn_qkv_conv1d_update_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ weight, const float* __restrict__ bias,
    uint16_t* __restrict__ state, const int32_t* __restrict__ slot_ids, int B, int pool, int C,
    QkvOut o) {
  const int c0 = 8 * (blockIdx.x * kConvThreads + threadIdx.x);
  if (c0 >= C) return;
  const int b0 = blockIdx.y * kUpdSeqs;
  float wt[8][W], bs[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    bs[e] = bias != nullptr ? bias[c0 + e] : 0.f;
#pragma unroll
    for (int j = 0; j < W; ++j) wt[e][j] = weight[(c0 + e) * W + j];
  }
  int slot[kUpdSeqs];
  bool live[kUpdSeqs];
  uint4 xw[kUpdSeqs], raw[kUpdSeqs][S];
#pragma unroll
  for (int u = 0; u < kUpdSeqs; ++u) {
    const int b = b0 + u;
    slot[u] = b < B ? (slot_ids != nullptr ? slot_ids[b] : b) : -1;
    live[u] = slot[u] >= 0 && slot[u] < pool;
    if (live[u]) {
      xw[u] = *reinterpret_cast<const uint4*>(x + size_t(b) * C + c0);
      // the lane's state block: channels c0 .. c0 + 7, S entries each, 16 S
      // contiguous bytes (S 16-byte words)
      const uint4* st = reinterpret_cast<const uint4*>(state + (size_t(slot[u]) * C + c0) * S);
#pragma unroll
      for (int i = 0; i < S; ++i) raw[u][i] = st[i];
    }
  }
#pragma unroll
  for (int u = 0; u < kUpdSeqs; ++u) {
    const int b = b0 + u;
    if (b >= B) break;
    float y[8];
    if (!live[u]) {
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = 0.f;
      store8(out_at(o, b, c0), y);
      continue;
    }
    float xc[8];
    unpack_bf16x2(xw[u].x, xc[0], xc[1]);
    unpack_bf16x2(xw[u].y, xc[2], xc[3]);
    unpack_bf16x2(xw[u].z, xc[4], xc[5]);
    unpack_bf16x2(xw[u].w, xc[6], xc[7]);
    auto elem = [&](int idx) {                // bf16 element idx of the block (idx constant)
      const uint4 w = raw[u][idx >> 3];
      const int q = idx & 7;
      const uint32_t d = (q >> 1) == 0 ? w.x : (q >> 1) == 1 ? w.y : (q >> 1) == 2 ? w.z : w.w;
      return (q & 1) ? (d >> 16) : (d & 0xffffu);
    };
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = bs[e];
#pragma unroll
      for (int j = 0; j < W - 1; ++j)   // window input j: state entry S - (W - 1) + j
        acc = fmaf(wt[e][j], bf16_bits_to_f32(elem(e * S + S - (W - 1) + j)), acc);
      acc = fmaf(wt[e][W - 1], xc[e], acc);
      y[e] = activate<kSilu>(acc);
    }
    store8(out_at(o, b, c0), y);
    // shifted block: entry si of channel e <- entry si + 1 (the token last)
    uint32_t nw[8 * S];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int si = 0; si < S; ++si)
        nw[e * S + si] = si + 1 < S ? elem(e * S + si + 1) : uint32_t(f32_to_bf16_bits(xc[e]));
    uint4* st = reinterpret_cast<uint4*>(state + (size_t(slot[u]) * C + c0) * S);
#pragma unroll
    for (int i = 0; i < S; ++i) {
      uint4 w;
      w.x = nw[8 * i + 0] | (nw[8 * i + 1] << 16);
      w.y = nw[8 * i + 2] | (nw[8 * i + 3] << 16);
      w.z = nw[8 * i + 4] | (nw[8 * i + 5] << 16);
      w.w = nw[8 * i + 6] | (nw[8 * i + 7] << 16);
      st[i] = w;
    }
  }
}

int check_qkv(const uint16_t* q, const uint16_t* k, const uint16_t* v, int C, int cq, int ck,
              QkvOut& o) {
  if (!q) return GDN_ERR_NULL;
  if (k == nullptr && v == nullptr) {         // one [tokens, C] output
    o = QkvOut{const_cast<uint16_t*>(q), nullptr, nullptr, C, 0, 0};
    return GDN_OK;
  }
  if (!k || !v) return GDN_ERR_NULL;
  if (cq <= 0 || ck <= 0 || cq % 8 || ck % 8 || cq + ck >= C) return GDN_ERR_SHAPE;
  o = QkvOut{const_cast<uint16_t*>(q), const_cast<uint16_t*>(k), const_cast<uint16_t*>(v), cq, ck,
             C - cq - ck};
  return GDN_OK;
}

template <typename CuT, bool kSilu>
void launch_conv(int W, dim3 grid, hipStream_t st, const uint16_t* x, const float* weight,
                 const float* bias, const CuT* cu, int N, int T, int C, const uint16_t* st_in,
                 uint16_t* st_out, int S, QkvOut o, int n_tiles) {
  switch (W) {
    case 2:
      hipLaunchKernelGGL((gdn_qkv_conv1d_kernel<2, CuT, kSilu>), grid, dim3(kConvThreads), 0, st, x, weight,
                         bias, cu, N, T, C, st_in, st_out, S, o, n_tiles);
      break;
    case 3:
      hipLaunchKernelGGL((gdn_qkv_conv1d_kernel<3, CuT, kSilu>), grid, dim3(kConvThreads), 0, st, x, weight,
                         bias, cu, N, T, C, st_in, st_out, S, o, n_tiles);
      break;
    default:
      hipLaunchKernelGGL((gdn_qkv_conv1d_kernel<4, CuT, kSilu>), grid, dim3(kConvThreads), 0, st, x, weight,
                         bias, cu, N, T, C, st_in, st_out, S, o, n_tiles);
      break;
  }
}

template <int W, bool kSilu>
void launch_update_w(int S, dim3 grid, hipStream_t st, const uint16_t* x, const float* weight,
                     const float* bias, uint16_t* state, const int32_t* slots, int B, int pool, int C,
                     QkvOut o) {
  if (S == W - 1)
    hipLaunchKernelGGL((gdn_qkv_conv1d_update_kernel<W, W - 1, kSilu>), grid, dim3(kConvThreads), 0, st, x,
                       weight, bias, state, slots, B, pool, C, o);
  else
    hipLaunchKernelGGL((gdn_qkv_conv1d_update_kernel<W, W, kSilu>), grid, dim3(kConvThreads), 0, st, x,
                       weight, bias, state, slots, B, pool, C, o);
}

template <bool kSilu>
void launch_update(int W, int S, dim3 grid, hipStream_t st, const uint16_t* x, const float* weight,
                   const float* bias, uint16_t* state, const int32_t* slots, int B, int pool, int C,
                   QkvOut o) {
  switch (W) {
    case 2: launch_update_w<2, kSilu>(S, grid, st, x, weight, bias, state, slots, B, pool, C, o); break;
    case 3: launch_update_w<3, kSilu>(S, grid, st, x, weight, bias, state, slots, B, pool, C, o); break;
    default: launch_update_w<4, kSilu>(S, grid, st, x, weight, bias, state, slots, B, pool, C, o); break;
  }
}

}  // namespace

extern "C" int gdn_qkv_conv1d_fwd(const uint16_t* x, const float* weight, const float* bias,
                                  const void* cu_seqlens, int cu_is_int32, int N, int T, int C,
                                  int W, const uint16_t* conv_state_in, uint16_t* conv_state_out,
                                  int state_len, uint16_t* out_q, uint16_t* out_k, uint16_t* out_v,
                                  int cq, int ck, int activation, void* stream) {
  if (N < 0 || T < 0 || C <= 0 || C % 8 || W < 2 || W > kMaxConvWidth) return GDN_ERR_SHAPE;
  if (state_len < W - 1 || state_len > kMaxStateLen) return GDN_ERR_SHAPE;
  if (activation != GDN_ACT_NONE && activation != GDN_ACT_SILU) return GDN_ERR_SHAPE;
  if (!cu_seqlens) return GDN_ERR_NULL;
  if (conv_state_out != nullptr && conv_state_out == conv_state_in) return GDN_ERR_SHAPE;
  if (N == 0 && T > 0) return GDN_ERR_SHAPE;   // tokens but no sequence to hold them
  if (T > 0 && (!x || !weight)) return GDN_ERR_NULL;
  if (N > 0 && conv_state_out != nullptr && !weight) return GDN_ERR_NULL;
  QkvOut o;
  if (T > 0) {
    const int rc = check_qkv(out_q, out_k, out_v, C, cq, ck, o);
    if (rc != GDN_OK) return rc;
  } else {
    o = QkvOut{out_q, out_k, out_v, C, 0, 0};
  }
  const int n_tiles = (T + kConvTile - 1) / kConvTile;
  const int rows = n_tiles + (conv_state_out != nullptr && N > 0 ? 1 : 0);
  if (rows == 0) return GDN_OK;
  const dim3 grid((C / 8 + kConvThreads - 1) / kConvThreads, rows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool silu = activation == GDN_ACT_SILU;
  if (cu_is_int32) {
    const int32_t* cu = static_cast<const int32_t*>(cu_seqlens);
    if (silu) launch_conv<int32_t, true>(W, grid, st, x, weight, bias, cu, N, T, C, conv_state_in, conv_state_out, state_len, o, n_tiles);
    else launch_conv<int32_t, false>(W, grid, st, x, weight, bias, cu, N, T, C, conv_state_in, conv_state_out, state_len, o, n_tiles);
  } else {
    const int64_t* cu = static_cast<const int64_t*>(cu_seqlens);
    if (silu) launch_conv<int64_t, true>(W, grid, st, x, weight, bias, cu, N, T, C, conv_state_in, conv_state_out, state_len, o, n_tiles);
    else launch_conv<int64_t, false>(W, grid, st, x, weight, bias, cu, N, T, C, conv_state_in, conv_state_out, state_len, o, n_tiles);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GDN_OK : -int(e);
}

extern "C" int gdn_qkv_conv1d_update(const uint16_t* x, const float* weight, const float* bias,
                                     uint16_t* conv_state, int state_len, const int32_t* slot_ids,
                                     int pool_size, int B, int C, int W, uint16_t* out_q,
                                     uint16_t* out_k, uint16_t* out_v, int cq, int ck,
                                     int activation, void* stream) {
  if (B < 0 || C <= 0 || C % 8 || W < 2 || W > kMaxConvWidth) return GDN_ERR_SHAPE;
  if (state_len != W - 1 && state_len != W) return GDN_ERR_SHAPE;
  if (activation != GDN_ACT_NONE && activation != GDN_ACT_SILU) return GDN_ERR_SHAPE;
  if (B == 0) return GDN_OK;
  if (!x || !weight || !conv_state) return GDN_ERR_NULL;
  if (slot_ids != nullptr ? pool_size < 0 : pool_size < B) return GDN_ERR_SHAPE;
  QkvOut o;
  const int rc = check_qkv(out_q, out_k, out_v, C, cq, ck, o);
  if (rc != GDN_OK) return rc;
  const dim3 grid((C / 8 + kConvThreads - 1) / kConvThreads, (B + kUpdSeqs - 1) / kUpdSeqs);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int pool = slot_ids != nullptr ? pool_size : B;
  if (activation == GDN_ACT_SILU) launch_update<true>(W, state_len, grid, st, x, weight, bias, conv_state, slot_ids, B, pool, C, o);
  else launch_update<false>(W, state_len, grid, st, x, weight, bias, conv_state, slot_ids, B, pool, C, o);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GDN_OK : -int(e);
}
