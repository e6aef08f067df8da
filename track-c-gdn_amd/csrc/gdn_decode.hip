// GDN decode: one recurrent step per (sequence, v-head), single pass over the
// fp32 k-last state.  Replaces the reference's Triton decode kernel
// (gdn_decode_qk4_v8_d128_k_last/solution/triton/kernel.py:26-79).
//
// Per (n, h), with S = state[n, h] in [V=128, K=128] (K contiguous):
//   S'    = g * S
//   delta = beta * (v - S' k)
//   S_new = S' + delta k^T
//   o     = scale * S_new q = scale * (S' q + delta (k . q))
//
// Mapping (gfx950, wave64):
//   * two workgroups of 4 waves per (n, v-head), 16 rows per wave; q/k are
//     read once per workgroup (they are 0.2% of the bytes).
//   * a DPP row (16 lanes) owns one state row; lane c holds k = 4c..4c+3 and
//     64+4c..64+4c+3, so each dwordx4 load covers four 256-byte row segments.
//   * each lane keeps 4 rows (8 x float4 = 128 B) in registers: all loads are
//     issued before any arithmetic, the row reductions are 4 DPP adds each,
//     and the updated row is written straight back (no LDS, no second pass).
//   * 63 VGPRs, so 8 waves per SIMD stream the state: the same bytes in
//     flight as 4 waves with 8 rows each, from twice as many waves.
//   * in-place update (state_in == state_out) is safe: every element is read
//     and written by the same lane.

#include "gdn_common.h"
#include "../../include/gdn_hip.h"

namespace {

using namespace gdn;

constexpr int D = kHeadDim;
constexpr int kWavesPerHead = 8;
constexpr int kRowsPerWave = D / kWavesPerHead;   // 16
constexpr int kRowsPerLane = kRowsPerWave / 4;    // 4 (4 DPP rows per wave)
constexpr int kThreadsPerHead = kWavesPerHead * kWave;
// Single-step decode: a head's 128 rows over kDecParts workgroups of
// kDecWaves waves (16 rows per wave).  Workgroups of 4 waves and 32 KB of
// state stream a 128 MiB state about 3.5% faster than 8 waves and 64 KB
// (the same rows per lane, measured with copies of either shape).
constexpr int kDecWaves = 4;
constexpr int kDecParts = kWavesPerHead / kDecWaves;
constexpr int kDecThreads = kDecWaves * kWave;
static_assert(kRowsPerLane == 4, "v is read and o written as 4 bf16 per lane");
constexpr int kTokBlock = 16;     // tokens staged in LDS at a time (multi-token decode)
// Multi-token decode: 2 state rows per lane, so a workgroup of 8 waves holds
// half a head (64 rows) and kMHeadParts = 2 workgroups share one (n, v-head).
constexpr int kMRowsPerLane = 2;
constexpr int kMHeadParts = kRowsPerLane / kMRowsPerLane;
constexpr int kMRowsPerWave = 4 * kMRowsPerLane;   // 4 DPP rows per wave

template <bool kNonTemporal>
__device__ __forceinline__ f32x4 load_state(const f32x4* p) {
  if constexpr (kNonTemporal) return __builtin_nontemporal_load(p);
  else return *p;
}

template <bool kNonTemporal>
__device__ __forceinline__ void store_state(f32x4* p, f32x4 x) {
  if constexpr (kNonTemporal) __builtin_nontemporal_store(x, p);
  else *p = x;
}

__device__ __forceinline__ void load_bf16x8_split(const uint16_t* base, int c, float (&x)[8]) {
  // elements 4c..4c+3 and 64+4c..64+4c+3
  const uint2 lo = *reinterpret_cast<const uint2*>(base + 4 * c);
  const uint2 hi = *reinterpret_cast<const uint2*>(base + 64 + 4 * c);
  unpack_bf16x2(lo.x, x[0], x[1]);
  unpack_bf16x2(lo.y, x[2], x[3]);
  unpack_bf16x2(hi.x, x[4], x[5]);
  unpack_bf16x2(hi.y, x[6], x[7]);
}

template <bool kNonTemporal, bool kL2>
__global__ __launch_bounds__(kDecThreads, kL2 ? 6 : 8) void gdn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* state_in, float* state_out,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    uint16_t* __restrict__ out, const int32_t* __restrict__ slot_ids,
    int HQ, int HV, int pool_size, float scale) {
  const int ratio = HV / HQ;
  const int head = blockIdx.x / kDecParts, part = blockIdx.x - head * kDecParts;
  const int n = head / HV;
  const int hv = head - n * HV;
  const int hq = hv / ratio;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row0 = (part * kDecWaves + wave) * kRowsPerWave;
  const int rsub = lane >> 4;     // DPP row within the wave
  const int c = lane & 15;        // lane within the DPP row
  const int rbase = row0 + rsub * kRowsPerLane;   // this lane's 8 consecutive rows

  const size_t nh = size_t(n) * HV + hv;
  uint16_t* o_ptr = out + nh * D + rbase;

  int slot = n;
  if (slot_ids != nullptr) {
    slot = slot_ids[n];
    if (slot < 0 || slot >= pool_size) {
      // Unmapped sequence: no state access, zero output.
      if (c == 0) *reinterpret_cast<uint2*>(o_ptr) = make_uint2(0, 0);
      return;
    }
  }
  const size_t sbase = (size_t(slot) * HV + hv) * size_t(D) * D;

  // Issue the state loads first: 16 x 16 B in flight per lane.
  f32x4 s[kRowsPerLane][2];
  if (state_in != nullptr) {
    const float* sp = state_in + sbase + size_t(rbase) * D;
#pragma unroll
    for (int j = 0; j < kRowsPerLane; ++j) {
      s[j][0] = load_state<kNonTemporal>(reinterpret_cast<const f32x4*>(sp + j * D + 4 * c));
      s[j][1] = load_state<kNonTemporal>(reinterpret_cast<const f32x4*>(sp + j * D + 64 + 4 * c));
    }
  } else {
#pragma unroll
    for (int j = 0; j < kRowsPerLane; ++j) {
      s[j][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      s[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  const size_t qk_off = (size_t(n) * HQ + hq) * D;
  float kk[8], qq[8];
  load_bf16x8_split(k + qk_off, c, kk);
  load_bf16x8_split(q + qk_off, c, qq);
  if constexpr (kL2) {      // option GDN_QK_L2NORM
    l2norm_row16(kk);
    l2norm_row16(qq);
  }
  float vv[kRowsPerLane];
  {
    const uint2 vw = *reinterpret_cast<const uint2*>(v + nh * D + rbase);
    unpack_bf16x2(vw.x, vv[0], vv[1]);
    unpack_bf16x2(vw.y, vv[2], vv[3]);
  }

  // Gates (reference DEC:59-65), uniform per wave.
  const float a_val = bf16_bits_to_f32(a[nh]);
  const float b_val = bf16_bits_to_f32(b[nh]);
  const float g = expf(-expf(A_log[hv]) * softplus_thresh20(a_val + dt_bias[hv]));
  const float beta = 1.0f / (1.0f + expf(-b_val));

  float kq = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) kq = fmaf(kk[e], qq[e], kq);
  kq = row16_sum(kq);

  float o_out[kRowsPerLane];
  float* dst = state_out + sbase + size_t(rbase) * D;
#pragma unroll
  for (int j = 0; j < kRowsPerLane; ++j) {
    float x[8] = {s[j][0].x, s[j][0].y, s[j][0].z, s[j][0].w,
                  s[j][1].x, s[j][1].y, s[j][1].z, s[j][1].w};
    float pk = 0.f, pq = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] *= g;
      pk = fmaf(x[e], kk[e], pk);
      pq = fmaf(x[e], qq[e], pq);
    }
    pk = row16_sum(pk);
    pq = row16_sum(pq);
    const float delta = beta * (vv[j] - pk);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = fmaf(delta, kk[e], x[e]);
    o_out[j] = scale * fmaf(delta, kq, pq);
    store_state<kNonTemporal>(reinterpret_cast<f32x4*>(dst + j * D + 4 * c),
                              f32x4{x[0], x[1], x[2], x[3]});
    store_state<kNonTemporal>(reinterpret_cast<f32x4*>(dst + j * D + 64 + 4 * c),
                              f32x4{x[4], x[5], x[6], x[7]});
  }
  if (c == 0) {
    uint2 w;
    w.x = pack_bf16x2(o_out[0], o_out[1]);
    w.y = pack_bf16x2(o_out[2], o_out[3]);
    *reinterpret_cast<uint2*>(o_ptr) = w;
  }
}

// Multi-token decode: T tokens of each sequence applied in order with the
// state held in registers in between (one state read and one state write for
// the T steps).  Token t of sequence n uses q, k [n, t, hq], v [n, t, hv] and
// a, b [n, t, hv]; its output goes to out [n, t, hv].  The per-token
// arithmetic is the single-step kernel's, in the same order, so T steps here
// give the same bits as T launches of gdn_decode_kernel.
template <bool kNonTemporal>
__global__ __launch_bounds__(kThreadsPerHead, 8) void gdn_decode_multi_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* state_in, float* state_out,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    uint16_t* __restrict__ out, int T, int HQ, int HV, float scale, int flags) {
  const int ratio = HV / HQ;
  const int part = blockIdx.x % kMHeadParts;
  const int nh = blockIdx.x / kMHeadParts;
  const int n = nh / HV;
  const int hv = nh - n * HV;
  const int hq = hv / ratio;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row0 = part * (D / kMHeadParts) + (wave % kWavesPerHead) * kMRowsPerWave;
  const int rsub = lane >> 4;
  const int c = lane & 15;
  const int rbase = row0 + rsub * kMRowsPerLane;
  const size_t sbase = (size_t(n) * HV + hv) * size_t(D) * D;

  f32x4 s[kMRowsPerLane][2];
  if (state_in != nullptr) {
    const float* sp = state_in + sbase + size_t(rbase) * D;
#pragma unroll
    for (int j = 0; j < kMRowsPerLane; ++j) {
      s[j][0] = load_state<kNonTemporal>(reinterpret_cast<const f32x4*>(sp + j * D + 4 * c));
      s[j][1] = load_state<kNonTemporal>(reinterpret_cast<const f32x4*>(sp + j * D + 64 + 4 * c));
    }
  } else {
#pragma unroll
    for (int j = 0; j < kMRowsPerLane; ++j) {
      s[j][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      s[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  const float a_log_exp = expf(A_log[hv]);
  const float dtb = dt_bias[hv];

  // Token inputs go through LDS in blocks of kTokBlock tokens, widened to
  // fp32 once: k, q and this head's v row (128 values each per token),
  // copied by the whole workgroup with 16-byte loads.  Then one 16-lane group
  // per token normalises k and q (option GDN_QK_L2NORM) and forms k.q, with
  // the lane layout and summation order of the single-step kernel (lane c:
  // elements 4c .. 4c+3 and 64+4c .. 64+4c+3), and one thread per token forms
  // the gates g, beta.  The serial token loop then only reads LDS.
  __shared__ __align__(16) float tk[kTokBlock][3][D];   // k | q | v
  __shared__ float tab[kTokBlock][3];                   // g, beta, k.q
  for (int t0 = 0; t0 < T; t0 += kTokBlock) {
    const int nt = min(kTokBlock, T - t0);
    __syncthreads();     // the previous block's reads are done
    for (int e = threadIdx.x; e < nt * 3 * (D / 8); e += kThreadsPerHead) {
      const int t = e / (3 * (D / 8)), r = e - t * (3 * (D / 8));
      const int which = r / (D / 8), chunk = r - which * (D / 8);
      const size_t tok = size_t(n) * T + t0 + t;
      const uint16_t* src = which == 0 ? k + (tok * HQ + hq) * D
                          : which == 1 ? q + (tok * HQ + hq) * D
                                       : v + (tok * HV + hv) * D;
      const uint4 w = *reinterpret_cast<const uint4*>(src + 8 * chunk);
      float x[8];
      unpack_bf16x2(w.x, x[0], x[1]); unpack_bf16x2(w.y, x[2], x[3]);
      unpack_bf16x2(w.z, x[4], x[5]); unpack_bf16x2(w.w, x[6], x[7]);
      *reinterpret_cast<f32x4*>(&tk[t][which][8 * chunk]) = f32x4{x[0], x[1], x[2], x[3]};
      *reinterpret_cast<f32x4*>(&tk[t][which][8 * chunk + 4]) = f32x4{x[4], x[5], x[6], x[7]};
    }
    if (int(threadIdx.x) < nt) {      // gates (reference DEC:59-65)
      const int t = threadIdx.x;
      const size_t tok = size_t(n) * T + t0 + t;
      tab[t][0] = expf(-a_log_exp * softplus_thresh20(bf16_bits_to_f32(a[tok * HV + hv]) + dtb));
      tab[t][1] = 1.0f / (1.0f + expf(-bf16_bits_to_f32(b[tok * HV + hv])));
    }
    __syncthreads();
    {
      const int t = 4 * wave + rsub;          // one 16-lane group per token
      if (t < nt) {
        float kk[8], qq[8];
        const f32x4 k0 = *reinterpret_cast<const f32x4*>(&tk[t][0][4 * c]);
        const f32x4 k1 = *reinterpret_cast<const f32x4*>(&tk[t][0][64 + 4 * c]);
        const f32x4 q0 = *reinterpret_cast<const f32x4*>(&tk[t][1][4 * c]);
        const f32x4 q1 = *reinterpret_cast<const f32x4*>(&tk[t][1][64 + 4 * c]);
        kk[0] = k0.x; kk[1] = k0.y; kk[2] = k0.z; kk[3] = k0.w;
        kk[4] = k1.x; kk[5] = k1.y; kk[6] = k1.z; kk[7] = k1.w;
        qq[0] = q0.x; qq[1] = q0.y; qq[2] = q0.z; qq[3] = q0.w;
        qq[4] = q1.x; qq[5] = q1.y; qq[6] = q1.z; qq[7] = q1.w;
        if (flags & GDN_QK_L2NORM) {
          l2norm_row16(kk);
          l2norm_row16(qq);
          *reinterpret_cast<f32x4*>(&tk[t][0][4 * c]) = f32x4{kk[0], kk[1], kk[2], kk[3]};
          *reinterpret_cast<f32x4*>(&tk[t][0][64 + 4 * c]) = f32x4{kk[4], kk[5], kk[6], kk[7]};
          *reinterpret_cast<f32x4*>(&tk[t][1][4 * c]) = f32x4{qq[0], qq[1], qq[2], qq[3]};
          *reinterpret_cast<f32x4*>(&tk[t][1][64 + 4 * c]) = f32x4{qq[4], qq[5], qq[6], qq[7]};
        }
        float kq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) kq = fmaf(kk[e], qq[e], kq);
        kq = row16_sum(kq);
        if (c == 0) tab[t][2] = kq;
      }
    }
    __syncthreads();
    for (int t = 0; t < nt; ++t) {
      float kk[8], vv[kMRowsPerLane];
      float qq[8];
      {
        const f32x4 k0 = *reinterpret_cast<const f32x4*>(&tk[t][0][4 * c]);
        const f32x4 k1 = *reinterpret_cast<const f32x4*>(&tk[t][0][64 + 4 * c]);
        const f32x4 q0 = *reinterpret_cast<const f32x4*>(&tk[t][1][4 * c]);
        const f32x4 q1 = *reinterpret_cast<const f32x4*>(&tk[t][1][64 + 4 * c]);
        const float2 vw = *reinterpret_cast<const float2*>(&tk[t][2][rbase]);
        kk[0] = k0.x; kk[1] = k0.y; kk[2] = k0.z; kk[3] = k0.w;
        kk[4] = k1.x; kk[5] = k1.y; kk[6] = k1.z; kk[7] = k1.w;
        qq[0] = q0.x; qq[1] = q0.y; qq[2] = q0.z; qq[3] = q0.w;
        qq[4] = q1.x; qq[5] = q1.y; qq[6] = q1.z; qq[7] = q1.w;
        vv[0] = vw.x; vv[1] = vw.y;
      }
      const float g = tab[t][0];
      const float beta = tab[t][1];
      const float kq = tab[t][2];
      float o_out[kMRowsPerLane];
#pragma unroll
      for (int j = 0; j < kMRowsPerLane; ++j) {
        float x[8] = {s[j][0].x, s[j][0].y, s[j][0].z, s[j][0].w,
                      s[j][1].x, s[j][1].y, s[j][1].z, s[j][1].w};
        float pk = 0.f, pq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[e] *= g;
          pk = fmaf(x[e], kk[e], pk);
          pq = fmaf(x[e], qq[e], pq);
        }
        pk = row16_sum(pk);
        pq = row16_sum(pq);
        const float delta = beta * (vv[j] - pk);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = fmaf(delta, kk[e], x[e]);
        o_out[j] = scale * fmaf(delta, kq, pq);
        s[j][0] = f32x4{x[0], x[1], x[2], x[3]};
        s[j][1] = f32x4{x[4], x[5], x[6], x[7]};
      }
      if (c == 0)
        *reinterpret_cast<uint32_t*>(out + ((size_t(n) * T + t0 + t) * HV + hv) * D + rbase) =
            pack_bf16x2(o_out[0], o_out[1]);
    }
  }
  float* dst = state_out + sbase + size_t(rbase) * D;
#pragma unroll
  for (int j = 0; j < kMRowsPerLane; ++j) {
    store_state<kNonTemporal>(reinterpret_cast<f32x4*>(dst + j * D + 4 * c), s[j][0]);
    store_state<kNonTemporal>(reinterpret_cast<f32x4*>(dst + j * D + 64 + 4 * c), s[j][1]);
  }
}

int check_decode_args(const void* q, const void* k, const void* v, const void* state_out,
                      const void* A_log, const void* a, const void* dt_bias, const void* b,
                      const void* out, int B, int HQ, int HV) {
  if (B < 0 || HQ <= 0 || HV <= 0 || HV % HQ != 0) return GDN_ERR_SHAPE;
  // An empty batch reads and writes nothing; its tensors may have no storage.
  if (B > 0 && (!q || !k || !v || !state_out || !A_log || !a || !dt_bias || !b || !out))
    return GDN_ERR_NULL;
  return GDN_OK;
}

int launch_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* state_in,
                  float* state_out, const float* A_log, const uint16_t* a, const float* dt_bias,
                  const uint16_t* b, uint16_t* out, const int32_t* slot_ids, int B, int HQ, int HV,
                  int pool_size, float scale, int flags, void* stream) {
  if (B == 0) return GDN_OK;
  const dim3 grid(unsigned(B) * unsigned(HV) * kDecParts);
  const dim3 block(kDecThreads);
  if (flags & GDN_QK_L2NORM)
    hipLaunchKernelGGL((gdn_decode_kernel<true, true>), grid, block, 0, static_cast<hipStream_t>(stream),
                       q, k, v, state_in, state_out, A_log, a, dt_bias, b, out, slot_ids, HQ, HV,
                       pool_size, scale);
  else
    hipLaunchKernelGGL((gdn_decode_kernel<true, false>), grid, block, 0, static_cast<hipStream_t>(stream),
                       q, k, v, state_in, state_out, A_log, a, dt_bias, b, out, slot_ids, HQ, HV,
                       pool_size, scale);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? GDN_OK : -int(err);
}

int launch_decode_multi(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        const float* state_in, float* state_out, const float* A_log,
                        const uint16_t* a, const float* dt_bias, const uint16_t* b, uint16_t* out,
                        int B, int T, int HQ, int HV, float scale, int flags, void* stream) {
  if (B == 0) return GDN_OK;
  const dim3 grid(unsigned(B) * unsigned(HV) * kMHeadParts);
  const dim3 block(kThreadsPerHead);
  hipLaunchKernelGGL(gdn_decode_multi_kernel<true>, grid, block, 0, static_cast<hipStream_t>(stream),
                     q, k, v, state_in, state_out, A_log, a, dt_bias, b, out, T, HQ, HV, scale,
                     flags);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? GDN_OK : -int(err);
}

}  // namespace

extern "C" int gdn_decode_multi_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    const float* state, float* new_state, const float* A_log,
                                    const uint16_t* a, const float* dt_bias, const uint16_t* b,
                                    uint16_t* out, int B, int T, int HQ, int HV, float scale,
                                    int flags, void* stream) {
  const int rc = check_decode_args(q, k, v, new_state, A_log, a, dt_bias, b, out, B, HQ, HV);
  if (rc != GDN_OK) return rc;
  if (T < 1) return GDN_ERR_SHAPE;
  if (flags & ~GDN_DECODE_FLAGS_ALL) return GDN_ERR_SHAPE;
  return launch_decode_multi(q, k, v, state, new_state, A_log, a, dt_bias, b, out, B, T, HQ, HV,
                             scale, flags, stream);
}

extern "C" int gdn_decode_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const float* state, float* new_state, const float* A_log,
                              const uint16_t* a, const float* dt_bias, const uint16_t* b,
                              uint16_t* out, int B, int HQ, int HV, float scale, void* stream) {
  const int rc = check_decode_args(q, k, v, new_state, A_log, a, dt_bias, b, out, B, HQ, HV);
  if (rc != GDN_OK) return rc;
  return launch_decode(q, k, v, state, new_state, A_log, a, dt_bias, b, out, nullptr, B, HQ, HV,
                       B, scale, 0, stream);
}

extern "C" int gdn_decode_ex_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const float* state, float* new_state, const float* A_log,
                                 const uint16_t* a, const float* dt_bias, const uint16_t* b,
                                 uint16_t* out, int B, int HQ, int HV, float scale, int flags,
                                 void* stream) {
  const int rc = check_decode_args(q, k, v, new_state, A_log, a, dt_bias, b, out, B, HQ, HV);
  if (rc != GDN_OK) return rc;
  if (flags & ~GDN_DECODE_FLAGS_ALL) return GDN_ERR_SHAPE;
  return launch_decode(q, k, v, state, new_state, A_log, a, dt_bias, b, out, nullptr, B, HQ, HV,
                       B, scale, flags, stream);
}

extern "C" int gdn_decode_pool_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                   float* state_pool, int pool_size, const int32_t* slot_ids,
                                   const float* A_log, const uint16_t* a, const float* dt_bias,
                                   const uint16_t* b, uint16_t* out, int B, int HQ, int HV,
                                   float scale, void* stream) {
  const int rc = check_decode_args(q, k, v, state_pool, A_log, a, dt_bias, b, out, B, HQ, HV);
  if (rc != GDN_OK) return rc;
  if (!slot_ids && B > 0) return GDN_ERR_NULL;
  if (pool_size < 0) return GDN_ERR_SHAPE;
  return launch_decode(q, k, v, state_pool, state_pool, A_log, a, dt_bias, b, out, slot_ids, B,
                       HQ, HV, pool_size, scale, 0, stream);
}
