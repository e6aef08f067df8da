// GDN chunked varlen prefill, backward (gfx950 / CDNA4, wave64, MFMA).
//
// The reference is forward-only (gdn_prefill_qk4_v8_d128_k_last/solution/
// triton/kernel.py:1); a training step needs the gradients of the prefill's
// inputs.  These kernels compute them from the states entering every chunk,
// h, which gdn_prefill_h_fwd writes (the h of the reference's
// chunk_gated_delta_rule_fwd_h, kernel.py:1153-1160).
//
// Per chunk (C = 64 rows, gam = chunk-local cumsum of the log-decay g,
// E = e^gam, Dc = e^{gam_L - gam}, S the state entering the chunk, dSn the
// gradient of the state leaving it) the forward is
//   Ar = tril_strict(e^{gam_i-gam_j} K K^T), A = diag(beta) Ar, Tm = (I + A)^-1,
//   P = scale tril_incl(e^{gam_i-gam_j} Q K^T), X = beta (V - E K S^T),
//   Vn = Tm X, O = scale E Q S^T + P Vn, S' = e^{gam_L} S + Vn^T Dc K,
// and its reverse is arranged in three launches:
//
//  1. gdn_bwd_prep_kernel, one workgroup per (chunk, v-head), all chunks at
//     once: the state-gradient transition of the chunk,
//        M = e^{gam_L} I - W2^T (beta E K),   W2 = Tm^T Dc K            [K x K]
//        R = dO^T (scale E Q) - G1^T (beta E K),  G1 = Tm^T P^T dO      [V x K]
//     so that dS = dSn M + R.  M is written as ready MFMA A-operand
//     fragments, R in the accumulator layout of the chain kernel.
//  2. gdn_bwd_chain_kernel, one workgroup per (sequence, v-head), or per
//     quarter of its state rows when the chains are few: walks the chunks
//     from last to first with dS^T in MFMA accumulators, storing dSn of
//     every chunk (bf16) and the gradient of the initial state.
//  3. gdn_bwd_grad_kernel, one workgroup per (chunk, qk-head), its v-heads
//     in turn: with S and dSn known, every gradient of the chunk:
//        dVn = P^T dO + Dc K dSn^T,  dX = Tm^T dVn,  dV = beta dX,
//        dP = dO Vn^T,  dTm = dVn X^T,  dA = -Tm^T dTm Tm^T (strictly lower),
//        dQ = scale E dO S + dPm K,
//        dK = Dc Vn dSn - beta E dX S + dPm^T Q + dAb K + dAb^T K,
//        dbeta = rowsum(dA Ar) + rowsum(dX (V - E K S^T)),
//        dgam  = rowsum - colsum of (dP P) and of (dA A) + scale E rowsum(Q (dO S))
//                - beta E rowsum(dX K S^T) - Dc rowsum(Vn K dSn^T)
//                (+ sum_i Dc rowsum(Vn K dSn^T) + e^{gam_L} <dSn, S> at gam_L),
//        dg = reverse cumsum of dgam within the chunk,
//     with dPm = scale e^{gam_i-gam_j} dP (j <= i), dAb = beta_i e^{gam_i-gam_j} dA.
//     dq / dk of the v-heads that share a qk-head are summed in registers,
//     in v-head order, and stored once.
//
// All products run on MFMA 16x16x32 bf16 with fp32 accumulation; the matrix
// operands live in LDS as bf16 rows of the form [m][r] and are read either
// straight (one 16-byte read: row m, reduction slots r) or through
// transposing LDS reads (ds_read_b64_tr_b16) when the product reduces over
// the other index.  Tm comes from an fp32 forward substitution.  Rows past a
// chunk's end are zero with beta = 0 and g = 0, which makes every one of
// their contributions vanish.  The waves of a workgroup exchange data only
// through LDS, so their barriers wait for LDS operations alone
// (lds_barrier): global loads and stores stay in flight across them.

#include "gdn_prefill_common.h"
#include "gdn_prefill_split.h"
#include "../../include/gdn_hip.h"

#include <algorithm>

namespace {

using namespace gdn;

constexpr int LDK = D + 8;           // [*][128] bf16 rows (272 B)
constexpr int LDC = C + 8;           // [*][64] bf16 rows (144 B)
constexpr int LDA = C + 4;           // [64][64] fp32 rows (272 B)
constexpr int kCB = C * LDK;         // elements of a [64][128] buffer
constexpr int kTB = C * LDC;         // elements of a [64][64] buffer
constexpr size_t kMBytes = size_t(D) * D * 2;   // M record (bf16 fragments)
constexpr size_t kRBytes = size_t(D) * D * 2;   // R record (bf16, accumulator layout)
constexpr size_t kHBytes = size_t(D) * D * 2;   // dSn record (bf16 [v][k])
constexpr int kGradThreads = 512;

typedef short i16x8_t __attribute__((ext_vector_type(8)));

// MFMA 16x16x32 operand (lane l: row / column m0 + l % 16, reduction slots
// r0 + 8 (l / 16) .. +7) of a bf16 matrix stored [m][r] (r contiguous).
__device__ __forceinline__ bf16x8_t op_mr(const uint16_t* base, int ld, int m0, int r0, int lane) {
  return ld16_bf(base + (m0 + (lane & 15)) * ld + r0 + 8 * (lane >> 4));
}

// The same operand of a bf16 matrix stored [r][m] (m contiguous) in LDS: lane
// j of each 16-lane group reads 4 elements of row r0 + 8 q + j / 4 at column
// m0 + 4 (j % 4); the transposing read hands lane i the elements of column
// m0 + i of rows r0 + 8 q .. +3, the second read those of the next 4 rows.
__device__ __forceinline__ bf16x8_t op_rm(const uint16_t* base, int ld, int m0, int r0, int lane) {
  const int j = lane & 15;
  const uint16_t* p = base + (r0 + 8 * (lane >> 4) + (j >> 2)) * ld + m0 + 4 * (j & 3);
  const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)p);
  const i16x4_t hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(p + 4 * ld));
  const i16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, v);
}

// Accumulator tile (lane l holds rows r0 + 4 (l / 16) + i, column c0 + l % 16)
// to a bf16 matrix stored [row][col] / transposed [col][row].
__device__ __forceinline__ void st_tile(uint16_t* base, int ld, int r0, int c0, const f32x4& x, int lane) {
  uint16_t* p = base + (r0 + 4 * (lane >> 4)) * ld + c0 + (lane & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i * ld] = f32_to_bf16_bits(x[i]);
}

// Sum over the 4 lane groups (same lane % 16) of a wave.
__device__ __forceinline__ float group4_sum(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// Gate data of one chunk in LDS: gam | beta | e^gam | e^{gam_L - gam} (64 each),
// then gam_L, e^{gam_L}.  Wave-0 work: lane t takes token t of the chunk.
constexpr int GB_GAM = 0, GB_BETA = C, GB_E = 2 * C, GB_DC = 3 * C, GB_L = 4 * C, GB_EL = 4 * C + 1;
constexpr int GB_SZ = 4 * C + 4;

// The gate inputs of token `lane` of the chunk (wave 0): loaded early, used
// by chunk_gates_calc once the chunk's rows are on their way.
struct GateIn {
  float a, b, dt, alog;
};

__device__ __forceinline__ GateIn gate_inputs(const float* A_log, const uint16_t* a, const float* dt_bias,
                                              const uint16_t* b, int HV, int hv, int t0, int len, int lane) {
  const size_t i = size_t(t0 + min(lane, len - 1)) * HV + hv;
  return GateIn{bf16_bits_to_f32(a[i]), bf16_bits_to_f32(b[i]), dt_bias[hv], A_log[hv]};
}

// g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b) per token (zero
// past the chunk end), the chunk-local cumsum gam, e^gam and e^{gam_L - gam},
// with the forward kernels' hardware exp2 / log2 forms.
__device__ __forceinline__ void chunk_gates_calc(const GateIn& in, int len, int lane, float* gb) {
  constexpr float kLog2e = 1.44269504088896341f, kLn2 = 0.69314718055994531f;
  float g = 0.f, be = 0.f;
  if (lane < len) {
    const float x = in.a + in.dt;
    const float sp = fmaxf(x, 0.f) + kLn2 * __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e));
    g = -__builtin_amdgcn_exp2f(in.alog * kLog2e) * sp;
    be = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-in.b * kLog2e));
  }
  const float gam = wave_inclusive_scan(g);
  const float gl = __shfl(gam, 63);
  gb[GB_GAM + lane] = gam;
  gb[GB_BETA + lane] = be;
  gb[GB_E + lane] = __builtin_amdgcn_exp2f(gam * kLog2e);
  gb[GB_DC + lane] = __builtin_amdgcn_exp2f((gl - gam) * kLog2e);
  if (lane == 0) {
    gb[GB_L] = gl;
    gb[GB_EL] = __builtin_amdgcn_exp2f(gl * kLog2e);
  }
}

// Rows [t0, t0 + len) of a [*, stride] bf16 tensor (128 columns) into a
// [64][LDK] LDS buffer, rows past len zero, in two steps so that the HBM
// reads of several tensors are in flight together: rows_fetch issues this
// thread's 16-byte reads (2 of the 1024 of a tensor, 512 threads), rows_store
// writes them.
__device__ __forceinline__ void rows_fetch(uint4 (&w)[2], const uint16_t* src, size_t stride, int t0,
                                           int len, int tid) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int x = tid + it * kGradThreads, r = x >> 4, cc = (x & 15) * 8;
    w[it] = r < len ? *reinterpret_cast<const uint4*>(src + size_t(t0 + r) * stride + cc)
                    : make_uint4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ void rows_store(uint16_t* dst, const uint4 (&w)[2], int tid) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int x = tid + it * kGradThreads, r = x >> 4, cc = (x & 15) * 8;
    *reinterpret_cast<uint4*>(dst + r * LDK + cc) = w[it];
  }
}

// A 128 x 128 bf16 state (rows of 256 B in HBM) into a [128][LDK] LDS buffer,
// in the same two steps (4 reads per thread).
__device__ __forceinline__ void state_fetch(uint4 (&w)[4], const uint16_t* src, int tid) {
#pragma unroll
  for (int it = 0; it < 4; ++it) w[it] = reinterpret_cast<const uint4*>(src)[tid + it * kGradThreads];
}

__device__ __forceinline__ void state_store(uint16_t* dst, const uint4 (&w)[4], int tid) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int x = tid + it * kGradThreads, r = x >> 4, cc = (x & 15) * 8;
    *reinterpret_cast<uint4*>(dst + r * LDK + cc) = w[it];
  }
}

// (I + A)^-1 of the strictly lower A = diag(beta) Ar (fp32 [64][LDA] in LDS,
// zero on and above the diagonal), one wave, in fp32:
//   * the four diagonal 16 x 16 blocks by forward substitution, lane l taking
//     column l % 16 of block l / 16:  x_r = delta_rc - beta_r sum_{m<r} Ar_rm x_m;
//   * the blocks below them block-row by block-row,
//     T_ij = -T_ii (sum_{j<=m<i} A_im T_mj), on fp32 MFMA 16x16x4, each
//     product's sum staged through sZ (16 x 17 floats).
// The fp32 blocks go to sT ([64][LDA]), the bf16 result (zero above the
// diagonal) to sTm [i][j].  The wave's LDS operations complete in order, so
// its own writes are visible to its later reads without a barrier.
__device__ __forceinline__ void unit_lower_inverse(const float* sAr, const float* gb, float* sT,
                                                   float* sZ, uint16_t* sTm, int lane) {
  const int bi = lane >> 4, c = lane & 15;
  {
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 16 * bi + r;
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < r; m += 4) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(&sAr[row * LDA + 16 * bi + m]);
        acc = fmaf(a4[0], x[m], acc);
        acc = fmaf(a4[1], x[m + 1], acc);
        acc = fmaf(a4[2], x[m + 2], acc);
        acc = fmaf(a4[3], x[m + 3], acc);
      }
      x[r] = (r == c ? 1.f : 0.f) - gb[GB_BETA + row] * acc;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 16 * bi + r;
      sT[row * LDA + 16 * bi + c] = x[r];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
        if (jb != bi) sTm[row * LDC + 16 * jb + c] = 0;
      sTm[row * LDC + 16 * bi + c] = f32_to_bf16_bits(x[r]);
    }
  }
  const int q = lane >> 4;
#pragma unroll
  for (int i = 1; i < 4; ++i) {
#pragma unroll
    for (int j = i - 1; j >= 0; --j) {
      f32x4 z = {0.f, 0.f, 0.f, 0.f};
      const float be = gb[GB_BETA + 16 * i + c];
#pragma unroll
      for (int m = j; m < i; ++m)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const float a = be * sAr[(16 * i + c) * LDA + 16 * m + 4 * s4 + q];
          const float b = sT[(16 * m + 4 * s4 + q) * LDA + 16 * j + c];
          z = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, z, 0, 0, 0);
        }
#pragma unroll
      for (int e = 0; e < 4; ++e) sZ[(4 * q + e) * 17 + c] = z[e];
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const float a = sT[(16 * i + c) * LDA + 16 * i + 4 * s4 + q];
        const float b = sZ[(4 * s4 + q) * 17 + c];
        t = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, t, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * i + 4 * q + e;
        sT[row * LDA + 16 * j + c] = -t[e];
        sTm[row * LDC + 16 * j + c] = f32_to_bf16_bits(-t[e]);
      }
    }
  }
}

// Decayed, masked K K^T (strict: Ar, fp32) or scaled Q K^T (inclusive: P,
// bf16) tile (ti, tj) of the chunk from K / Q rows in LDS.
template <bool kP>
__device__ __forceinline__ void kk_tile(const uint16_t* sX, const uint16_t* sK, const float* gb, int ti,
                                        int tj, float scale, float* sAr, uint16_t* sP, int lane) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < D / 32; ++s)
    acc = mfma16_bf(op_mr(sX, LDK, 16 * ti, 32 * s, lane), op_mr(sK, LDK, 16 * tj, 32 * s, lane), acc);
  const int col = 16 * tj + (lane & 15);
  const float gc = gb[GB_GAM + col];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * ti + 4 * (lane >> 4) + i;
    const bool keep = kP ? row >= col : row > col;
    const float v = keep ? acc[i] * expf(gb[GB_GAM + row] - gc) : 0.f;
    if constexpr (kP) sP[row * LDC + col] = f32_to_bf16_bits(scale * v);
    else sAr[row * LDA + col] = v;
  }
}

// The 20 tiles of Ar and P on or below the diagonal, spread over 8 waves.
__device__ __forceinline__ void ar_p_tiles(const uint16_t* sK, const uint16_t* sQ, const float* gb,
                                           float scale, float* sAr, uint16_t* sP, int wave, int lane) {
  for (int job = wave; job < 20; job += 8) {
    const int t = job % 10;
    const int ti = t < 1 ? 0 : t < 3 ? 1 : t < 6 ? 2 : 3;
    const int tj = t - (ti * (ti + 1)) / 2;
    if (job < 10) kk_tile<false>(sK, sK, gb, ti, tj, scale, sAr, sP, lane);
    else kk_tile<true>(sQ, sK, gb, ti, tj, scale, sAr, sP, lane);
  }
}

// ---------------------------------------------------------------------------
// 1. Transition of the state gradient per (chunk, v-head): M and R.
//
// M record: 32 fragments of 1 KB, fragment (kt, s) = kt * 4 + s holds for
// lane l the 8 bf16 of M^T[16 kt + l % 16][j] at j = 32 s + 16 (e / 4) +
// 4 (l / 16) + e % 4, e = 0..7: the A operand of the chain kernel's product
// dS^T M-side, whose B operand is two stacked accumulator tiles of dS^T.
// R record: R^T tiles (kt, vt), vt-major, lane l's 4 values (bf16, 8 bytes)
// at 8 l: rows 16 kt + 4 (l / 16) + i, column 16 vt + l % 16 -- the chain
// kernel's accumulator layout.  bf16 like M and like the dSn operand the
// chain multiplies by M: R enters dS = dSn M + R with the same rounding.
template <typename CuT>
__global__ __launch_bounds__(kGradThreads, 1) void gdn_bwd_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const float* __restrict__ A_log,
    const uint16_t* __restrict__ a, const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    const CuT* __restrict__ cu, int N, int T, int HQ, int HV, float scale,
    const uint16_t* __restrict__ d_out, int h_chunks, int slots, char* __restrict__ mrec,
    char* __restrict__ rrec) {
  __shared__ __align__(16) uint16_t sK[kCB];      // K; then G0 = P^T dO
  __shared__ __align__(16) uint16_t sQ[kCB];      // Q; then W2 = Tm^T Dc K
  __shared__ __align__(16) uint16_t sdO[kCB];
  __shared__ __align__(16) uint16_t sDK[kCB];     // Dc K
  __shared__ __align__(16) uint16_t sBEK[kCB];    // beta E K
  __shared__ __align__(16) uint16_t sEQ[kCB];     // scale E Q
  __shared__ __align__(16) float sAr[C * LDA];    // Ar; then -G1 (bf16 [64][LDK])
  __shared__ __align__(16) uint16_t sP[kTB];
  __shared__ __align__(16) uint16_t sTm[kTB];
  __shared__ __align__(16) float sT[C * LDA];     // fp32 Tm blocks (the inverse's own)
  __shared__ __align__(16) float sZ[16 * 17];
  __shared__ __align__(16) float gb[GB_SZ];

  const int tid0 = threadIdx.x, lane0 = tid0 & 63;
  const int tid = tid0, lane = lane0;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Persistent workgroups (one per CU: the LDS holds one): workgroup w takes
  // the (chunk slot, v-head) units w, w + gridDim.x, ... (slot fastest, the
  // order of a (slots, HV) grid) and fetches the next unit's rows and gate
  // inputs into registers while it works on one, so the HBM latency of a
  // unit's inputs is spent inside the unit before it.
  const int units = slots * HV;
  auto locate = [&](int u, int& t0, int& len) {
    const int slot = u % slots;
    if (slot >= h_chunks) return false;
    int n, ci;
    locate_chunk(cu, N, T, slot, lane, n, ci);
    if (n < 0) return false;
    int bos, slen;
    seq_bounds(cu, n, T, bos, slen);
    t0 = bos + C * ci;
    len = min(C, slen - C * ci);
    return true;
  };
  auto fetch = [&](int u, int t0, int len, uint4 (&wk)[2], uint4 (&wq)[2], uint4 (&wo)[2], GateIn& gi) {
    const int hv = u / slots, hq = hv / (HV / HQ);
    if (wave == 0) gi = gate_inputs(A_log, a, dt_bias, b, HV, hv, t0, len, lane);
    rows_fetch(wk, k + size_t(hq) * D, size_t(HQ) * D, t0, len, tid);
    rows_fetch(wq, q + size_t(hq) * D, size_t(HQ) * D, t0, len, tid);
    rows_fetch(wo, d_out + size_t(hv) * D, size_t(HV) * D, t0, len, tid);
  };
  uint4 wk[2], wq[2], wo[2];
  GateIn gi{};
  int t0 = 0, len = 0;
  bool ok = int(blockIdx.x) < units && locate(int(blockIdx.x), t0, len);
  if (ok) fetch(int(blockIdx.x), t0, len, wk, wq, wo, gi);
  for (int u = int(blockIdx.x); u < units; u += int(gridDim.x)) {
    // the next unit's inputs, in flight while this one is worked on
    const int un = u + int(gridDim.x);
    int t0n = 0, lenn = 0;
    const bool okn = un < units && locate(un, t0n, lenn);
    uint4 wkn[2], wqn[2], won[2];
    GateIn gin{};
    if (okn) fetch(un, t0n, lenn, wkn, wqn, won, gin);
    if (ok) {
      const int slot = u % slots, hv = u / slots;
      // Lane indices opaque to the compiler at the top of each unit: their
      // address arithmetic is formed where it is used instead of being
      // hoisted out of the loop into registers live across every unit.
      int tid = tid0, lane = lane0;
      asm volatile("" : "+v"(tid), "+v"(lane));
      for (int x = tid; x < C * LDA; x += kGradThreads) sAr[x] = 0.f;
      for (int x = tid; x < kTB; x += kGradThreads) sP[x] = 0;
      rows_store(sK, wk, tid);
      rows_store(sQ, wq, tid);
      rows_store(sdO, wo, tid);
      if (wave == 0) chunk_gates_calc(gi, len, lane, gb);
      lds_barrier();

      // Ar, P; the scaled row copies
      ar_p_tiles(sK, sQ, gb, scale, sAr, sP, wave, lane);
      for (int x = tid; x < C * 16; x += kGradThreads) {
        const int r = x >> 4, cc = (x & 15) * 8;
        const uint4 kw = *reinterpret_cast<const uint4*>(&sK[r * LDK + cc]);
        const uint4 qw = *reinterpret_cast<const uint4*>(&sQ[r * LDK + cc]);
        const float fd = gb[GB_DC + r], fb = gb[GB_BETA + r] * gb[GB_E + r], fq = scale * gb[GB_E + r];
        const uint32_t kk[4] = {kw.x, kw.y, kw.z, kw.w}, qq[4] = {qw.x, qw.y, qw.z, qw.w};
        uint32_t od[4], ob[4], oq[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float k0, k1, q0, q1;
          unpack_bf16x2(kk[e], k0, k1);
          unpack_bf16x2(qq[e], q0, q1);
          od[e] = pack_bf16x2(fd * k0, fd * k1);
          ob[e] = pack_bf16x2(fb * k0, fb * k1);
          oq[e] = pack_bf16x2(fq * q0, fq * q1);
        }
        *reinterpret_cast<uint4*>(&sDK[r * LDK + cc]) = make_uint4(od[0], od[1], od[2], od[3]);
        *reinterpret_cast<uint4*>(&sBEK[r * LDK + cc]) = make_uint4(ob[0], ob[1], ob[2], ob[3]);
        *reinterpret_cast<uint4*>(&sEQ[r * LDK + cc]) = make_uint4(oq[0], oq[1], oq[2], oq[3]);
      }
      lds_barrier();

      // Tm (wave 0) while waves 1-7 form G0 = P^T dO [t][v] over sK (K is done)
      if (wave == 0) {
        unit_lower_inverse(sAr, gb, sT, sZ, sTm, lane);
      } else {
        for (int x = wave - 1; x < 32; x += 7) {
          const int tb = x & 3, vb = x >> 2;
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < C / 32; ++s)
            acc = mfma16_bf(op_rm(sP, LDC, 16 * tb, 32 * s, lane), op_rm(sdO, LDK, 16 * vb, 32 * s, lane), acc);
          st_tile(sK, LDK, 16 * tb, 16 * vb, acc, lane);
        }
      }
      lds_barrier();

      // W2 = Tm^T Dc K -> sQ, -G1 = -Tm^T G0 -> sAr (as bf16 [64][LDK])
      uint16_t* sG1 = reinterpret_cast<uint16_t*>(sAr);
      {
        const int tb = wave & 3, d0 = 4 * (wave >> 2);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int db = d0 + u;
          f32x4 w2 = {0.f, 0.f, 0.f, 0.f}, g1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < C / 32; ++s) {
            const bf16x8_t tmt = op_rm(sTm, LDC, 16 * tb, 32 * s, lane);
            w2 = mfma16_bf(tmt, op_rm(sDK, LDK, 16 * db, 32 * s, lane), w2);
            g1 = mfma16_bf(tmt, op_rm(sK, LDK, 16 * db, 32 * s, lane), g1);
          }
          st_tile(sQ, LDK, 16 * tb, 16 * db, w2, lane);
          st_tile(sG1, LDK, 16 * tb, 16 * db, -g1, lane);
        }
      }
      lds_barrier();

      // M = e^{gam_L} I - W2^T (beta E K): tiles (jt, kt); R^T = (scale E Q)^T dO + (beta E K)^T (-G1)
      const size_t rec = size_t(slot) * HV + hv;
      char* mr = mrec + rec * kMBytes;
      char* rr = rrec + rec * kRBytes;
      const float eL = gb[GB_EL];
      {
        const int jt = wave;
#pragma unroll 2
        for (int kt = 0; kt < 8; ++kt) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < C / 32; ++s)
            acc = mfma16_bf(op_rm(sQ, LDK, 16 * jt, 32 * s, lane), op_rm(sBEK, LDK, 16 * kt, 32 * s, lane), acc);
          const int kcol = 16 * kt + (lane & 15);
          float m[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int jrow = 16 * jt + 4 * (lane >> 4) + i;
            m[i] = (jrow == kcol ? eL : 0.f) - acc[i];
          }
          uint2 w;
          w.x = pack_bf16x2(m[0], m[1]);
          w.y = pack_bf16x2(m[2], m[3]);
          *reinterpret_cast<uint2*>(mr + ((kt * 4 + (jt >> 1)) * 64 + lane) * 16 + 8 * (jt & 1)) = w;
        }
        const int kt = wave;
#pragma unroll 2
        for (int vt = 0; vt < 8; ++vt) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < C / 32; ++s) {
            acc = mfma16_bf(op_rm(sEQ, LDK, 16 * kt, 32 * s, lane), op_rm(sdO, LDK, 16 * vt, 32 * s, lane), acc);
            acc = mfma16_bf(op_rm(sBEK, LDK, 16 * kt, 32 * s, lane), op_rm(sG1, LDK, 16 * vt, 32 * s, lane), acc);
          }
          *reinterpret_cast<uint2*>(rr + ((vt * 8 + kt) * 64 + lane) * 8) =
              uint2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
        }
      }
      // the next unit overwrites every buffer this one reads last
      lds_barrier();
    }
    ok = okn;
    t0 = t0n;
    len = lenn;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      wk[i] = wkn[i];
      wq[i] = wqn[i];
      wo[i] = won[i];
    }
    gi = gin;
  }
}

// ---------------------------------------------------------------------------
// 2. The state-gradient chain per (sequence, v-head), last chunk first:
//    dh[chunk] = dSn (bf16 [v][k]);  dS = dSn M + R;  finally dh0 = dS.
// NW waves per workgroup, 128 / (16 NW) workgroups per chain.  A wave keeps
// dS^T[k][v] for its 16 state rows v as 8 accumulator tiles (k blocks); the
// B operand of step s is the pair of tiles kt = 2 s, 2 s + 1.
template <typename CuT, int NW>
__global__ __launch_bounds__(64 * NW, 1) void gdn_bwd_chain_kernel(
    const CuT* __restrict__ cu, int N, int T, int HV, int h_chunks, const char* __restrict__ mrec,
    const char* __restrict__ rrec, const float* __restrict__ d_ht, uint16_t* __restrict__ dh,
    float* __restrict__ dh0) {
  constexpr int S = 8 / NW;                    // slices (of 16 NW state rows) per chain
  constexpr int kThreads = 64 * NW;
  __shared__ __align__(16) uint16_t sM[3][D * D];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup -> (chain = (sequence, v-head), slice).  The rows of dS evolve
  // independently (dS = dSn M + R row by row), so a chain splits over S
  // workgroups that never exchange data; its slices get ids 8 apart, which
  // puts them on one XCD, so M is read from HBM once per chain.
  const int xcd = blockIdx.x & 7, id_row = blockIdx.x >> 3;
  const int chain = 8 * (id_row / S) + xcd;
  if (chain >= N * HV) return;
  const int slice = id_row - (id_row / S) * S;
  const int n = chain / HV, hv = chain - n * HV;
  int bos, slen;
  seq_bounds(cu, n, T, bos, slen);
  const int nc = (slen + C - 1) / C;
  const int coff = chunk_offset(cu, n, T, lane);
  const int g = lane >> 4, c = lane & 15;
  const int vb = slice * NW + wave;            // 16-row block of the state this wave holds
  const int v = 16 * vb + c;                   // state row (v) of this lane's accumulator column

  f32x4 acc[8];
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) {
    const int k0 = 16 * kt + 4 * g;
    acc[kt] = d_ht ? *reinterpret_cast<const f32x4*>(d_ht + ((size_t(n) * HV + hv) * D + v) * D + k0)
                   : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  int last = nc - 1;
  if (coff + last >= h_chunks) last = -1;     // records at or past h_chunks (clamped to the workspace's slots) were not formed
  // M is copied HBM -> LDS and R loaded into registers two chunks ahead: three
  // LDS buffers for M and three register sets for R, rotated by unrolling the
  // chunk loop by three.
  constexpr int kMCopies = int(kMBytes / 16) / kThreads;
  auto rec_of = [&](int ch) { return size_t(coff + ch) * HV + hv; };
  auto copy_m = [&](int ch, int buf) {
    const char* ms = mrec + rec_of(ch) * kMBytes;
#pragma unroll
    for (int x = 0; x < kMCopies; ++x)
      lds_dma16_saddr(ms, uint32_t((x * kThreads + tid) * 16), &sM[buf][(x * kThreads + wave * 64) * 8]);
  };
  auto fetch_r = [&](int ch, uint2 (&r)[8]) {
    const char* rs = rrec + rec_of(ch) * kRBytes;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      r[kt] = *reinterpret_cast<const uint2*>(rs + ((vb * 8 + kt) * 64 + lane) * 8);
  };
  // one chunk: dSn out, dS = dSn M + R (cur = R of chunk ch), and the copies
  // for chunk ch - 2 (R into nxt2, M into LDS buffer (it + 2) % 3)
  auto step = [&](int ch, int it, uint2 (&cur)[8], uint2 (&nxt2)[8]) {
    const int buf = it % 3;
    if (ch > 1) {
      copy_m(ch - 2, (it + 2) % 3);
      fetch_r(ch - 2, nxt2);
    }
    uint16_t* hd = dh + rec_of(ch) * D * D;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      uint2 w;
      w.x = pack_bf16x2(acc[kt][0], acc[kt][1]);
      w.y = pack_bf16x2(acc[kt][2], acc[kt][3]);
      *reinterpret_cast<uint2*>(hd + v * D + 16 * kt + 4 * g) = w;
    }
    bf16x8_t bop[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) bop[s] = pack2_bf(acc[2 * s], acc[2 * s + 1]);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      acc[kt] = f32x4{__uint_as_float(cur[kt].x << 16), __uint_as_float(cur[kt].x & 0xffff0000u),
                      __uint_as_float(cur[kt].y << 16), __uint_as_float(cur[kt].y & 0xffff0000u)};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        acc[kt] = mfma16_bf(ld16_bf(&sM[buf][((kt * 4 + s) * 64 + lane) * 8]), bop[s], acc[kt]);
    }
    // Vector memory operations complete in issue order: with at most this
    // chunk's copies (M and R two chunks ahead) and its 8 dSn stores still
    // outstanding, everything the next chunk reads has landed.
    if (ch > 1) wait_vm<kMCopies + 8 + 8>();
    else wait_vm<8>();
    lds_barrier();
  };
  uint2 r0[8], r1[8], r2[8];
  if (last >= 0) {
    copy_m(last, 0);
    fetch_r(last, r0);
    if (last > 0) {
      copy_m(last - 1, 1);
      fetch_r(last - 1, r1);
    }
  }
  wait_vm<0>();
  lds_barrier();
  for (int ch = last, it = 0; ch >= 0; ch -= 3, it += 3) {
    step(ch, it, r0, r2);
    if (ch >= 1) step(ch - 1, it + 1, r1, r0);
    if (ch >= 2) step(ch - 2, it + 2, r2, r1);
  }
  if (dh0) {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      *reinterpret_cast<f32x4*>(dh0 + ((size_t(n) * HV + hv) * D + v) * D + 16 * kt + 4 * g) = acc[kt];
  }
}

// ---------------------------------------------------------------------------
// 3. Gradients of one (chunk, v-head) given S (h) and dSn (the chain's dh).
// [64][128] products: wave w owns row block tb = w % 4 and column blocks
// 4 (w / 4) .. +3.  [64][64] products: row block ib = w / 2, column blocks
// 2 (w % 2), +1.  Row and column sums of the dgam / dbeta terms go through
// per-contributor partial arrays (fixed summation order).
struct GradParts {
  float ag[2][C];    // dgam rows, [64][128] products (contributor w / 4)
  float ab[2][C];    // dbeta rows, [64][128] products
  float vk[2][C];    // Dc rowsum(Vn K dSn^T)
  float tg[2][C];    // dgam rows, [64][64] products (contributor w % 2)
  float tb[2][C];    // dbeta rows, [64][64] products
  float tc[4][C];    // dgam column sums (to subtract), [64][64] products (contributor w / 2)
  float dot[8];      // <dSn, S> per wave
};

template <typename CuT>
__global__ __launch_bounds__(kGradThreads, 1) void gdn_bwd_grad_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a, const float* __restrict__ dt_bias,
    const uint16_t* __restrict__ b, const CuT* __restrict__ cu, int N, int T, int HQ, int HV,
    float scale, const uint16_t* __restrict__ d_out, const uint16_t* __restrict__ h, int h_chunks,
    const uint16_t* __restrict__ dh, float* __restrict__ dq, float* __restrict__ dk,
    float* __restrict__ dv, float* __restrict__ dg, float* __restrict__ dbeta) {
  __shared__ __align__(16) uint16_t sK_rows[kCB];
  __shared__ __align__(16) uint16_t sQ_rows[kCB];
  __shared__ __align__(16) uint16_t sdO[kCB];
  __shared__ __align__(16) uint16_t sVn[kCB];
  __shared__ __align__(16) uint16_t sX[kCB];      // V; X; then -beta E dX
  __shared__ __align__(16) uint16_t sS[2 * kCB];  // dVn | Ar (fp32); then S, dSn [128][LDK]
  __shared__ __align__(16) uint16_t sTm[kTB];     // Tm; then dPm
  __shared__ __align__(16) uint16_t sP[kTB];
  __shared__ __align__(16) uint16_t sdT[kTB];     // dTm; then dAb
  __shared__ __align__(16) uint16_t sY[kTB];
  __shared__ __align__(16) float gb[GB_SZ];
  __shared__ GradParts pt;
  uint16_t* sdV = sS;
  float* sAr = reinterpret_cast<float*>(sS + kCB);

  int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int g4 = lane >> 4, c16 = lane & 15;
  // One (chunk, qk-head) per workgroup: its G v-heads in turn, dq and dk
  // summed over them in registers (v-head order) and stored once.
  const int slot = blockIdx.x, hq = blockIdx.y;
  const int G = HV / HQ;
  if (slot >= h_chunks) return;
  int n, ci;
  locate_chunk(cu, N, T, slot, lane, n, ci);
  if (n < 0) return;
  int bos, slen;
  seq_bounds(cu, n, T, bos, slen);
  const int t0 = bos + C * ci;
  const int len = min(C, slen - C * ci);
  uint4 wk[2], wq[2];
  rows_fetch(wk, k + size_t(hq) * D, size_t(HQ) * D, t0, len, tid);
  rows_fetch(wq, q + size_t(hq) * D, size_t(HQ) * D, t0, len, tid);
  rows_store(sK_rows, wk, tid);
  rows_store(sQ_rows, wq, tid);
  const int tb = wave & 3, d0 = 4 * (wave >> 2);
  const int ib = wave >> 1, j0 = 2 * (wave & 1);
  f32x4 dq_acc[4], dk_acc[4];     // this wave's dq / dk tiles, summed over the v-heads

  for (int m = 0; m < G; ++m) {
  // K and Q rows stay in LDS across the v-heads; an offset the compiler
  // cannot see through (zero) keeps their reads inside the iteration, where
  // the registers are, instead of hoisted out of the loop.
  int lds0 = 0;
  asm volatile("" : "+s"(lds0));
  uint16_t* sK = sK_rows + lds0;
  uint16_t* sQ = sQ_rows + lds0;
  // likewise the lane indices: their address arithmetic is formed where it is used
  asm volatile("" : "+v"(tid), "+v"(lane), "+v"(g4), "+v"(c16));
  const int hv = hq * G + m;
  const size_t rec = (size_t(slot) * HV + hv) * D * D;
  const uint16_t* Sg = h + rec;
  const uint16_t* dSg = dh + rec;

  GateIn gi{};
  if (wave == 0) gi = gate_inputs(A_log, a, dt_bias, b, HV, hv, t0, len, lane);
  uint4 wo[2], wv[2];
  rows_fetch(wo, d_out + size_t(hv) * D, size_t(HV) * D, t0, len, tid);
  rows_fetch(wv, v + size_t(hv) * D, size_t(HV) * D, t0, len, tid);
  // the previous v-head's last reads of these buffers are behind the barrier
  // that ends its iteration
  for (int x = tid; x < C * LDA; x += kGradThreads) sAr[x] = 0.f;
  for (int x = tid; x < kTB; x += kGradThreads) sP[x] = 0;
  rows_store(sdO, wo, tid);
  rows_store(sX, wv, tid);
  if (wave == 0) chunk_gates_calc(gi, len, lane, gb);
  lds_barrier();

  ar_p_tiles(sK, sQ, gb, scale, sAr, sP, wave, lane);
  lds_barrier();

  f32x4 eks[4], xr[4], kds[4];
  // the inverse's fp32 blocks over sVn, its staging over sY (both unused until later)
  if (wave == 0) unit_lower_inverse(sAr, gb, reinterpret_cast<float*>(sVn), reinterpret_cast<float*>(sY), sTm, lane);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int db = d0 + u;
    f32x4 ks = {0.f, 0.f, 0.f, 0.f}, kd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      const bf16x8_t ko = op_mr(sK, LDK, 16 * tb, 32 * s, lane);
      ks = mfma16_bf(ko, op_mr(Sg, D, 16 * db, 32 * s, lane), ks);
      kd = mfma16_bf(ko, op_mr(dSg, D, 16 * db, 32 * s, lane), kd);
    }
    kds[u] = kd;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * tb + 4 * g4 + i;
      eks[u][i] = gb[GB_E + row] * ks[i];
      xr[u][i] = bf16_bits_to_f32(sX[row * LDK + 16 * db + c16]) - eks[u][i];
    }
  }
  lds_barrier();
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    f32x4 x;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = gb[GB_BETA + 16 * tb + 4 * g4 + i] * xr[u][i];
    st_tile(sX, LDK, 16 * tb, 16 * (d0 + u), x, lane);
  }
  lds_barrier();

  // Vn = Tm X;  dVn = Dc K dSn^T + P^T dO
  f32x4 vn[4];
  float vkp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int db = d0 + u;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < C / 32; ++s)
      x = mfma16_bf(op_mr(sTm, LDC, 16 * tb, 32 * s, lane), op_rm(sX, LDK, 16 * db, 32 * s, lane), x);
    vn[u] = x;
    st_tile(sVn, LDK, 16 * tb, 16 * db, x, lane);
    f32x4 y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      y[i] = gb[GB_DC + 16 * tb + 4 * g4 + i] * kds[u][i];
      vkp[i] = fmaf(x[i], kds[u][i], vkp[i]);
    }
#pragma unroll
    for (int s = 0; s < C / 32; ++s)
      y = mfma16_bf(op_rm(sP, LDC, 16 * tb, 32 * s, lane), op_rm(sdO, LDK, 16 * db, 32 * s, lane), y);
    st_tile(sdV, LDK, 16 * tb, 16 * db, y, lane);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float t = row16_sum(vkp[i]);
    const int row = 16 * tb + 4 * g4 + i;
    if (c16 == 0) pt.vk[wave >> 2][row] = gb[GB_DC + row] * t;
  }
  lds_barrier();

  // dX = Tm^T dVn (dV, dbeta / dgam terms);  dTm = dVn X^T
  f32x4 dx[4];
  float dgr[4] = {0.f, 0.f, 0.f, 0.f}, dbr[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int db = d0 + u;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < C / 32; ++s)
      x = mfma16_bf(op_rm(sTm, LDC, 16 * tb, 32 * s, lane), op_rm(sdV, LDK, 16 * db, 32 * s, lane), x);
    dx[u] = x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * tb + 4 * g4 + i;
      const float be = gb[GB_BETA + row];
      dbr[i] = fmaf(x[i], xr[u][i], dbr[i]);
      dgr[i] = fmaf(-be * x[i], eks[u][i], dgr[i]);
      if (row < len) dv[(size_t(t0 + row) * HV + hv) * D + 16 * db + c16] = be * x[i];
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
      x = mfma16_bf(op_mr(sdV, LDK, 16 * ib, 32 * s, lane), op_mr(sX, LDK, 16 * (j0 + u), 32 * s, lane), x);
    st_tile(sdT, LDC, 16 * ib, 16 * (j0 + u), x, lane);
  }
  lds_barrier();

  // -beta E dX -> sX;  Y = dTm Tm^T
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    f32x4 x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * tb + 4 * g4 + i;
      x[i] = -gb[GB_BETA + row] * gb[GB_E + row] * dx[u][i];
    }
    st_tile(sX, LDK, 16 * tb, 16 * (d0 + u), x, lane);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < C / 32; ++s)
      x = mfma16_bf(op_mr(sdT, LDC, 16 * ib, 32 * s, lane), op_mr(sTm, LDC, 16 * (j0 + u), 32 * s, lane), x);
    st_tile(sY, LDC, 16 * ib, 16 * (j0 + u), x, lane);
  }
  lds_barrier();

  // dA = -Tm^T Y (strictly lower), dP = dO Vn^T (inclusive lower): their dbeta / dgam terms
  uint4 wst[4];
  state_fetch(wst, Sg, tid);
  f32x4 dab[2], dpm[2];
  {
    float rg[4] = {0.f, 0.f, 0.f, 0.f}, rb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int jb = j0 + u;
      f32x4 da = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < C / 32; ++s)
        da = mfma16_bf(op_rm(sTm, LDC, 16 * ib, 32 * s, lane), op_rm(sY, LDC, 16 * jb, 32 * s, lane), da);
#pragma unroll
      for (int s = 0; s < D / 32; ++s)
        dp = mfma16_bf(op_mr(sdO, LDK, 16 * ib, 32 * s, lane), op_mr(sVn, LDK, 16 * jb, 32 * s, lane), dp);
      const int col = 16 * jb + c16;
      const float gc = gb[GB_GAM + col];
      float cs = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * ib + 4 * g4 + i;
        const float ex = row >= col ? expf(gb[GB_GAM + row] - gc) : 0.f;
        const float dA = row > col ? -da[i] : 0.f;
        const float dP = row >= col ? dp[i] : 0.f;
        const float ar = sAr[row * LDA + col];
        const float be = gb[GB_BETA + row];
        const float pv = bf16_bits_to_f32(sP[row * LDC + col]);
        const float aa = dA * be * ar, pp = dP * pv;
        rb[i] = fmaf(dA, ar, rb[i]);
        rg[i] += aa + pp;
        cs += aa + pp;
        dab[u][i] = be * ex * dA;
        dpm[u][i] = scale * ex * dP;
      }
      cs = group4_sum(cs);
      if (g4 == 0) pt.tc[ib][col] = cs;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float tg = row16_sum(rg[i]), tbv = row16_sum(rb[i]);
      const int row = 16 * ib + 4 * g4 + i;
      if (c16 == 0) {
        pt.tg[wave & 1][row] = tg;
        pt.tb[wave & 1][row] = tbv;
      }
    }
  }
  lds_barrier();
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    st_tile(sdT, LDC, 16 * ib, 16 * (j0 + u), dab[u], lane);
    st_tile(sTm, LDC, 16 * ib, 16 * (j0 + u), dpm[u], lane);
  }
  // S -> LDS [v][LDK] over dVn and Ar (both read for the last time above)
  state_store(sS, wst, tid);
  lds_barrier();

  // dQ = scale E dO S + dPm K;  dK (all but the dSn term) = -beta E dX S + dPm^T Q + dAb K + dAb^T K
  uint4 wds[4];
  state_fetch(wds, dSg, tid);
  f32x4 dkp[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int kb = d0 + u;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
      x = mfma16_bf(op_mr(sdO, LDK, 16 * tb, 32 * s, lane), op_rm(sS, LDK, 16 * kb, 32 * s, lane), x);
    f32x4 y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * tb + 4 * g4 + i;
      y[i] = scale * gb[GB_E + row] * x[i];
      dgr[i] = fmaf(y[i], bf16_bits_to_f32(sQ[row * LDK + 16 * kb + c16]), dgr[i]);
    }
#pragma unroll
    for (int s = 0; s < C / 32; ++s)
      y = mfma16_bf(op_mr(sTm, LDC, 16 * tb, 32 * s, lane), op_rm(sK, LDK, 16 * kb, 32 * s, lane), y);
    if (m == 0) dq_acc[u] = y;
    else dq_acc[u] += y;
    f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
      z = mfma16_bf(op_mr(sX, LDK, 16 * tb, 32 * s, lane), op_rm(sS, LDK, 16 * kb, 32 * s, lane), z);
#pragma unroll
    for (int s = 0; s < C / 32; ++s) {
      const bf16x8_t kop = op_rm(sK, LDK, 16 * kb, 32 * s, lane);
      z = mfma16_bf(op_rm(sTm, LDC, 16 * tb, 32 * s, lane), op_rm(sQ, LDK, 16 * kb, 32 * s, lane), z);
      z = mfma16_bf(op_mr(sdT, LDC, 16 * tb, 32 * s, lane), kop, z);
      z = mfma16_bf(op_rm(sdT, LDC, 16 * tb, 32 * s, lane), kop, z);
    }
    dkp[u] = z;
  }
  {
    // <dSn, S>: this thread's 32 elements of S (in LDS) against those of dSn
    float part = 0.f;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int x = tid + it * kGradThreads, r = x >> 4, cc = (x & 15) * 8;
      const uint4 sw = *reinterpret_cast<const uint4*>(&sS[r * LDK + cc]);
      const uint32_t ss[4] = {sw.x, sw.y, sw.z, sw.w};
      const uint32_t dd[4] = {wds[it].x, wds[it].y, wds[it].z, wds[it].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float s0, s1, d0, d1;
        unpack_bf16x2(ss[j], s0, s1);
        unpack_bf16x2(dd[j], d0, d1);
        part = fmaf(s0, d0, fmaf(s1, d1, part));
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
    if (lane == 0) pt.dot[wave] = part;
  }
  lds_barrier();
  state_store(sS, wds, tid);
  lds_barrier();

  // dK += Dc Vn dSn
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int kb = d0 + u;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
      x = mfma16_bf(op_mr(sVn, LDK, 16 * tb, 32 * s, lane), op_rm(sS, LDK, 16 * kb, 32 * s, lane), x);
    f32x4 z;
#pragma unroll
    for (int i = 0; i < 4; ++i) z[i] = fmaf(gb[GB_DC + 16 * tb + 4 * g4 + i], x[i], dkp[u][i]);
    if (m == 0) dk_acc[u] = z;
    else dk_acc[u] += z;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float tg = row16_sum(dgr[i]), tbv = row16_sum(dbr[i]);
    const int row = 16 * tb + 4 * g4 + i;
    if (c16 == 0) {
      pt.ag[wave >> 2][row] = tg;
      pt.ab[wave >> 2][row] = tbv;
    }
  }
  lds_barrier();

  if (wave == 0) {
    const int t = lane;
    const float vk = pt.vk[0][t] + pt.vk[1][t];
    float dgam = pt.ag[0][t] + pt.ag[1][t] - vk + pt.tg[0][t] + pt.tg[1][t] -
                 ((pt.tc[0][t] + pt.tc[1][t]) + (pt.tc[2][t] + pt.tc[3][t]));
    float vks = vk;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) vks += __shfl_xor(vks, off);
    float dot = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) dot += pt.dot[w];
    if (t == C - 1) dgam += vks + gb[GB_EL] * dot;
    // dg_t = sum_{i >= t} dgam_i
    const float incl = wave_inclusive_scan(dgam);
    const float total = __shfl(incl, 63);
    const float dgt = total - incl + dgam;
    const float dbt = (pt.ab[0][t] + pt.ab[1][t]) + (pt.tb[0][t] + pt.tb[1][t]);
    if (t < len) {
      dg[size_t(t0 + t) * HV + hv] = dgt;
      dbeta[size_t(t0 + t) * HV + hv] = dbt;
    }
  }
  lds_barrier();    // the next v-head rewrites every buffer but sK, sQ
  }

#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * tb + 4 * g4 + i;
      if (row < len) {
        const size_t at = (size_t(t0 + row) * HQ + hq) * D + 16 * (d0 + u) + c16;
        dq[at] = dq_acc[u][i];
        dk[at] = dk_acc[u][i];
      }
    }
}

// Gradients of the gating, per v-head (one workgroup each):
//   g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)
//   da = dg (-exp(A_log) sigmoid(a + dt_bias)),  ddt_bias = sum_t da,
//   dA_log = sum_t dg g,  db = dbeta beta (1 - beta).
__global__ __launch_bounds__(256) void gdn_gate_bwd_kernel(
    const float* __restrict__ A_log, const uint16_t* __restrict__ a, const float* __restrict__ dt_bias,
    const uint16_t* __restrict__ b, const float* __restrict__ dg, const float* __restrict__ dbeta, int T,
    int HV, float* __restrict__ da, float* __restrict__ db, float* __restrict__ dA_log,
    float* __restrict__ ddt_bias) {
  __shared__ float red[2][4];
  const int hv = blockIdx.x, tid = threadIdx.x;
  const float ea = expf(A_log[hv]), bias = dt_bias[hv];
  float sa = 0.f, sd = 0.f;
  for (int t = tid; t < T; t += 256) {
    const size_t i = size_t(t) * HV + hv;
    const float x = bf16_bits_to_f32(a[i]) + bias;
    const float g = dg[i];
    const float dai = -g * ea * sigmoidf_(x);
    const float be = sigmoidf_(bf16_bits_to_f32(b[i]));
    da[i] = dai;
    db[i] = dbeta[i] * be * (1.f - be);
    sa = fmaf(g, -ea * softplus_stable(x), sa);
    sd += dai;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sa += __shfl_xor(sa, off);
    sd += __shfl_xor(sd, off);
  }
  if ((tid & 63) == 0) {
    red[0][tid >> 6] = sa;
    red[1][tid >> 6] = sd;
  }
  __syncthreads();
  if (tid == 0) {
    dA_log[hv] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    ddt_bias[hv] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  }
}

template <typename CuT>
int launch_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* A_log,
               const uint16_t* a, const float* dt_bias, const uint16_t* b, const CuT* cu, int N, int T,
               int HQ, int HV, float scale, const uint16_t* h, int h_chunks, const uint16_t* d_out,
               const float* d_ht, float* dq, float* dk, float* dv, float* dg, float* dbeta, float* dh0,
               char* ws, hipStream_t st) {
  const size_t slots = size_t(T) / C + size_t(N);
  // The workspace holds `slots` chunk records per v-head.  Well-formed
  // cu_seqlens give at most that many chunks; with overlapping ranges the
  // chunk count (and h_chunks) can exceed it, and every kernel then stops at
  // the last slot the workspace holds (results unspecified, accesses in bounds).
  h_chunks = int(std::min<size_t>(size_t(h_chunks), slots));
  char* mrec = ws;
  char* rrec = mrec + slots * HV * kMBytes;
  uint16_t* dhr = reinterpret_cast<uint16_t*>(rrec + slots * HV * kRBytes);
  // Persistent workgroups, one per CU, when each takes many units (the next
  // unit's inputs are then fetched during the current one); with few units
  // per CU, one workgroup per unit, which the dispatcher balances.
  const int cus = device_cus();
  const size_t units = slots * size_t(HV);
  const size_t wgs = size_t(cus > 0 ? cus : 256);
  const unsigned pgrid = unsigned(units >= 8 * wgs ? wgs : units);
  hipLaunchKernelGGL((gdn_bwd_prep_kernel<CuT>), dim3(pgrid), dim3(kGradThreads), 0, st, q, k, A_log, a,
                     dt_bias, b, cu, N, T, HQ, HV, scale, d_out, h_chunks, int(slots), mrec, rrec);
  // The reverse chain: one workgroup of 8 waves per chain, or, when the
  // chains leave most CUs idle, 4 workgroups of 2 waves (32 state rows) each.
  const unsigned chain_ids = 8u * ((unsigned(N) * unsigned(HV) + 7u) / 8u);
  if (cus > 0 && 4LL * N * HV <= cus)
    hipLaunchKernelGGL((gdn_bwd_chain_kernel<CuT, 2>), dim3(4u * chain_ids), dim3(128), 0, st, cu, N, T,
                       HV, h_chunks, mrec, rrec, d_ht, dhr, dh0);
  else
    hipLaunchKernelGGL((gdn_bwd_chain_kernel<CuT, 8>), dim3(chain_ids), dim3(512), 0, st, cu, N, T, HV,
                       h_chunks, mrec, rrec, d_ht, dhr, dh0);
  if (T > 0) {
    // one workgroup per (chunk, qk-head), its v-heads in turn
    const dim3 qgrid{unsigned(slots), unsigned(HQ), 1u};
    hipLaunchKernelGGL((gdn_bwd_grad_kernel<CuT>), qgrid, dim3(kGradThreads), 0, st, q, k, v, A_log, a,
                       dt_bias, b, cu, N, T, HQ, HV, scale, d_out, h, h_chunks, dhr, dq, dk, dv, dg, dbeta);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GDN_OK : -int(e);
}

}  // namespace

extern "C" size_t gdn_prefill_bwd_workspace_bytes(int N, int T, int HQ, int HV) {
  if (N < 0 || T < 0 || HQ <= 0 || HV <= 0 || HV % HQ != 0) return 0;
  const size_t slots = size_t(T) / C + size_t(N);
  return slots * size_t(HV) * (kMBytes + kRBytes + kHBytes);
}

extern "C" int gdn_prefill_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const float* A_log, const uint16_t* a, const float* dt_bias,
                               const uint16_t* b, const void* cu_seqlens, int cu_is_int32, int N,
                               int T, int HQ, int HV, float scale, const uint16_t* h, int h_chunks,
                               const uint16_t* d_out, const float* d_final_state, float* dq, float* dk,
                               float* dv, float* dg, float* dbeta, float* d_initial_state,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (N < 0 || T < 0 || HQ <= 0 || HV <= 0 || HV % HQ != 0 || h_chunks < 0) return GDN_ERR_SHAPE;
  if (!cu_seqlens) return GDN_ERR_NULL;
  if (N > 0 && (!A_log || !dt_bias)) return GDN_ERR_NULL;
  if (T > 0 && (!q || !k || !v || !a || !b || !d_out || !dq || !dk || !dv || !dg || !dbeta))
    return GDN_ERR_NULL;
  if (h_chunks > 0 && !h) return GDN_ERR_NULL;
  if (N == 0) return GDN_OK;
  if (!workspace || workspace_bytes < gdn_prefill_bwd_workspace_bytes(N, T, HQ, HV))
    return GDN_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (cu_is_int32)
    return launch_bwd(q, k, v, A_log, a, dt_bias, b, static_cast<const int32_t*>(cu_seqlens), N, T, HQ,
                      HV, scale, h, h_chunks, d_out, d_final_state, dq, dk, dv, dg, dbeta,
                      d_initial_state, ws, st);
  return launch_bwd(q, k, v, A_log, a, dt_bias, b, static_cast<const int64_t*>(cu_seqlens), N, T, HQ, HV,
                    scale, h, h_chunks, d_out, d_final_state, dq, dk, dv, dg, dbeta, d_initial_state, ws,
                    st);
}

extern "C" int gdn_gate_bwd(const float* A_log, const uint16_t* a, const float* dt_bias, const uint16_t* b,
                            const float* dg, const float* dbeta, int T, int HV, float* da, float* db,
                            float* dA_log, float* ddt_bias, void* stream) {
  if (T < 0 || HV <= 0) return GDN_ERR_SHAPE;
  if (!A_log || !dt_bias || !dA_log || !ddt_bias) return GDN_ERR_NULL;
  if (T > 0 && (!a || !b || !dg || !dbeta || !da || !db)) return GDN_ERR_NULL;
  hipLaunchKernelGGL(gdn_gate_bwd_kernel, dim3(unsigned(HV)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     A_log, a, dt_bias, b, dg, dbeta, T, HV, da, db, dA_log, ddt_bias);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GDN_OK : -int(e);
}
