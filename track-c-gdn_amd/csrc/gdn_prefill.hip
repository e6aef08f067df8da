// GDN chunked varlen prefill, one fused kernel (gfx950 / CDNA4, wave64, MFMA).
//
// Replaces the reference prefill pipeline (five Triton launches plus host
// metadata; gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py
// :1570-1633, 1728-1759, 1762-1802).  One workgroup owns one
// (sequence, v-head) chain and walks its 64-token chunks in order; the fp32
// state S [V=128, K=128] never leaves registers between chunks, and nothing
// but q/k/v/a/b is read and o / final state written.
//
// Per chunk (C = 64 rows, gam = chunk-local cumsum of the log-decay,
// S = state at chunk start), the same mathematics as the reference
// (kernel.py:509-525, 661-796, 1153-1339, 1447-1496) arranged so that W and U
// are never formed:
//   A   = tril_strict(beta_i e^{gam_i-gam_j} K K^T)      (MFMA 16x16x32)
//   P   = tril_incl(e^{gam_i-gam_j} Q K^T)                (MFMA 16x16x32)
//   Tm  = (I + A)^-1      (fp32 16x16 diagonal blocks, MFMA block merges)
//   X   = diag(beta) (V - diag(e^gam) K S^T)               (MFMA 32x32x16)
//   Vn  = Tm X          ( = U - W S^T of the reference )   (MFMA 32x32x16)
//   O   = scale (diag(e^gam) Q S^T + P Vn)                 (MFMA 32x32x16)
//   S  <- e^{gam_L} S + (diag(e^{gam_L-gam}) Vn)^T K       (MFMA 32x32x16)
// MFMA operands are fp16 (bf16 inputs convert exactly in fp16's normal
// range; fp16 keeps 3 more mantissa bits than bf16 for the fp32 state and
// intermediates), accumulation is fp32.
//
// Wave w of the 4 waves owns state rows v in [32w, 32w+32): every product
// that touches S, X, Vn or O is split along v, so the waves never exchange
// state.  The state lives as S^T accumulator tiles; because an MFMA reduces
// over an arbitrary pairing of its 16 k-slots, each accumulator tile is used
// directly as the B operand of the next product (k-slot e of lane half h is
// row 16s + 8(e/4) + 4h + e%4 of the tile), with the A operand read from LDS
// in the matching order: no cross-lane shuffles, only fp32->fp16 packs.

#include "gdn_common.h"
#include "../../include/gdn_hip.h"

namespace {

using namespace gdn;

constexpr int D = kHeadDim;   // 128
constexpr int C = 64;         // chunk
constexpr int KLD = D + 8;    // sK / sQ row stride (halves): 272 B rows
constexpr int TLD = C + 8;    // sKT / sTm / sP row stride (halves): 144 B rows
constexpr int ALD = C + 4;    // sA row stride (floats): 272 B rows
constexpr int kThreads = 256; // 4 waves, one per SIMD

typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

// Column order inside every 16-column group of the fp16 operand tiles: the
// two middle quads are swapped (bits 2 and 3 of the index), so that the 8
// k-slots lane half h feeds an MFMA -- rows {0-3, 8-11} (h = 0) or
// {4-7, 12-15} (h = 1) of a 16-row accumulator block -- are 16 contiguous
// bytes.  The map is its own inverse.
__device__ __forceinline__ int perm16(int c) { return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1); }

// LDS written by DMA lives in objects of its own, so that the compiler can
// tell the other LDS accesses from the in-flight DMA writes.
struct __align__(16) SmemRaw {
  uint16_t k[C * D];           // next chunk's K rows as loaded (bf16)
  uint16_t q[C * D];           // next chunk's Q rows as loaded (bf16)
};

struct __align__(16) Smem {
  _Float16 K[C * KLD];         // K chunk [t][perm(k)]
  _Float16 Q[C * KLD];         // Q chunk [t][perm(k)]
  _Float16 KT[D * TLD];        // K chunk transposed [k][perm(t)]
  _Float16 Tm[C * TLD];        // (I + A)^-1 [t][perm(t')]
  _Float16 P[C * TLD];         // decayed causal Q K^T [t][perm(t')]
  float A[C * ALD];            // beta-scaled decayed strict K K^T [t][t'] (fp32)
  float gam[2][C];             // chunk-local cumsum of the log-decay (double-buffered)
  float beta[2][C];
  float eg[2][C];              // e^{gam_t}
  float ed[2][C];              // e^{gam_{L-1} - gam_t}
};

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for its outstanding global loads or HBM->LDS DMA (those are
// waited for explicitly where their data is consumed).  The asm statement is
// a compiler memory barrier as well.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ f16x8 ld16(const _Float16* p) { return *reinterpret_cast<const f16x8*>(p); }

__device__ __forceinline__ f16x8 ld_f32x8_as_f16(const float* p) {
  const f32x4 lo = *reinterpret_cast<const f32x4*>(p);
  const f32x4 hi = *reinterpret_cast<const f32x4*>(p + 4);
  return f16x8{(_Float16)lo[0], (_Float16)lo[1], (_Float16)lo[2], (_Float16)lo[3],
               (_Float16)hi[0], (_Float16)hi[1], (_Float16)hi[2], (_Float16)hi[3]};
}

__device__ __forceinline__ f16x8 pack8(const f32x16& x, int s) {
  f16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (_Float16)x[8 * s + e];
  return r;
}

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16k16(f16x4_t a, f16x4_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Row of accumulator element i for lane half h (32x32 layout).
__device__ __forceinline__ int acc_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// HBM -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane l's
// bytes land at lds_dst + 16 l; lds_dst must be uniform across the wave.
// Issued from asm so that the compiler does not wait for it at the next LDS
// access it cannot disambiguate; every consumer of the copied data waits for
// it explicitly (vmcnt) and then crosses a barrier.
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_dst) {
  const uint32_t lds_addr = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds_dst);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_addr), "v"(src) : "memory");
}

template <typename CuT>
__global__ __launch_bounds__(kThreads, 1) void gdn_prefill_chain_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ h0,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    const CuT* __restrict__ cu_seqlens, int T, int HQ, int HV, float scale,
    uint16_t* __restrict__ out, float* __restrict__ ht) {
  __shared__ Smem sm;
  __shared__ SmemRaw raw;
  __shared__ __align__(16) uint16_t rawV[C * D];    // V chunk (bf16) [t][v], filled by DMA

  const int n = blockIdx.x / HV;
  const int hv = blockIdx.x - n * HV;
  const int hq = hv / (HV / HQ);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int h = lane >> 5;        // lane half (32x32 MFMA layouts)
  const int col = lane & 31;
  const int g4 = lane >> 4;       // lane group (16x16 MFMA layouts)
  const int c16 = lane & 15;
  const int vrow = 32 * wave + col;   // state row v owned by this lane

  long long bos_l = (long long)cu_seqlens[n];
  long long eos_l = (long long)cu_seqlens[n + 1];
  bos_l = bos_l < 0 ? 0 : (bos_l > T ? T : bos_l);
  eos_l = eos_l < bos_l ? bos_l : (eos_l > T ? T : eos_l);
  const int bos = int(bos_l);
  const int len = int(eos_l - bos_l);

  const float a_log_exp = expf(A_log[hv]);
  const float dtb = dt_bias[hv];
  const size_t qk_stride = size_t(HQ) * D;   // elements per token in q / k
  const size_t v_stride = size_t(HV) * D;    // elements per token in v / out
  const int n_chunks = (len + C - 1) / C;

  // Upper 16x16 tiles inside the diagonal 32x32 blocks of Tm / P are read by
  // the 32x32 products and must be zero; they are never written afterwards.
  for (int e = tid; e < 2 * 16 * 16; e += kThreads) {
    const int blk = e >> 8, r = (e >> 4) & 15, c = e & 15;
    const int R = 32 * blk + r, Cc = 32 * blk + 16 + c;
    sm.Tm[R * TLD + Cc] = (_Float16)0.f;
    sm.P[R * TLD + Cc] = (_Float16)0.f;
  }

  // Wave w owns chunk rows [16w, 16w+16) of the staging: it DMAs them from
  // HBM into rawK / rawQ / rawV one chunk ahead and converts the same K / Q
  // rows, so no other wave touches its raw rows in between.  Lane l of DMA
  // instruction r carries row 16w + 4r + l/16, columns 8(l%16)..+7; rows past
  // the chunk end are clamped to its last row (zeroed at conversion).
  uint16_t ra = 0, rb = 0;            // gate inputs of row `lane` (wave 1)
  // K / Q rows of chunk ch (issued once this wave has converted the previous
  // chunk's raw rows) and the gate inputs of chunk ch (wave 1).
  auto issue_kq = [&](int ch) {
    const int t0 = bos + ch * C;
    const int L = min(C, len - ch * C);
    if (wave == 1) {
      const size_t gi = size_t(t0 + min(lane, L - 1)) * HV + hv;
      ra = a[gi];
      rb = b[gi];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row0 = 16 * wave + 4 * r;
      const int row = min(row0 + (lane >> 4), L - 1);
      const size_t off = size_t(t0 + row) * qk_stride + size_t(hq) * D + (lane & 15) * 8;
      lds_dma16(k + off, &raw.k[row0 * D]);
      lds_dma16(q + off, &raw.q[row0 * D]);
    }
  };
  // V rows of chunk ch (issued once every wave has read the previous chunk's V).
  auto issue_v = [&](int ch) {
    const int t0 = bos + ch * C;
    const int L = min(C, len - ch * C);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row0 = 16 * wave + 4 * r;
      const int row = min(row0 + (lane >> 4), L - 1);
      lds_dma16(v + size_t(t0 + row) * v_stride + size_t(hv) * D + (lane & 15) * 8, &rawV[row0 * D]);
    }
  };
  // Gates of chunk ch (wave 1): log-decay, its inclusive scan, beta, decays.
  auto gates_chunk = [&](int ch) {
    const int L = min(C, len - ch * C);
    const int gb = ch & 1;
    float ld = 0.f, bt = 0.f;
    if (lane < L) {
      ld = -a_log_exp * softplus_stable(bf16_bits_to_f32(ra) + dtb);
      bt = sigmoidf_(bf16_bits_to_f32(rb));
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(ld, off, 64);
      if (lane >= off) ld += y;
    }
    const float gl = __shfl(ld, L - 1, 64);
    sm.gam[gb][lane] = ld;
    sm.beta[gb][lane] = bt;
    sm.eg[gb][lane] = expf(ld);
    sm.ed[gb][lane] = expf(gl - ld);
  };

  // ---- initial state: S^T tiles, Sacc[j][i] = S[vrow][32j + acc_row(i, h)]
  f32x16 Sacc[4];
  const size_t state_off = (size_t(n) * HV + hv) * size_t(D) * D + size_t(vrow) * D;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (h0 != nullptr) x = *reinterpret_cast<const f32x4*>(h0 + state_off + 32 * j + 8 * g + 4 * h);
      Sacc[j][4 * g + 0] = x[0];
      Sacc[j][4 * g + 1] = x[1];
      Sacc[j][4 * g + 2] = x[2];
      Sacc[j][4 * g + 3] = x[3];
    }
  }

  if (n_chunks > 0) {
    issue_kq(0);
    if (wave == 1) gates_chunk(0);
    issue_v(0);
  }
  // Output of the previous chunk, packed bf16 pairs in accumulator order: it
  // is stored at the start of the next chunk, so that no recent store sits
  // in front of the waits for the DMA.
  uint32_t opack[2][8];
  int o_t0 = 0;

  for (int ch = 0; ch < n_chunks; ++ch) {
    const int t0 = bos + ch * C;
    const int L = min(C, len - ch * C);
    const uint16_t* sV = rawV;
    const int gb = ch & 1;
    const float* g_gam = sm.gam[gb];
    const float* g_beta = sm.beta[gb];
    const float* g_eg = sm.eg[gb];
    const float* g_ed = sm.ed[gb];

    // ================= P0: convert this wave's raw rows; gates; prefetch ch+1
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's DMA of chunk ch landed
    if (ch > 0) {
      // output of chunk ch-1 (a full chunk: only the last chunk can be ragged).
      // Row 32tt + 8g + 4h + r: a uniform row pointer plus a per-lane offset.
      const uint32_t loff = uint32_t(vrow) + uint32_t(4 * h) * uint32_t(v_stride);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = 4 * g + r;
            uint16_t* rowp = out + size_t(o_t0 + 32 * tt + 8 * g + r) * v_stride + size_t(hv) * D;
            rowp[loff] = uint16_t(opack[tt][i >> 1] >> (16 * (i & 1)));
          }
        }
      }
    }
    {
      const int r0 = 16 * wave + 4 * g4;          // this lane's quad of rows
      const int cc = c16 * 8;                     // and its 8 columns
      const int pc_lo = (cc & ~15) + ((cc & 8) ? 4 : 0);
      float kf[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool valid = r0 + r < L;
        uint4 kw = *reinterpret_cast<const uint4*>(&raw.k[(r0 + r) * D + cc]);
        uint4 qw = *reinterpret_cast<const uint4*>(&raw.q[(r0 + r) * D + cc]);
        if (!valid) { kw = make_uint4(0, 0, 0, 0); qw = make_uint4(0, 0, 0, 0); }
        float qf[8];
        unpack_bf16x2(kw.x, kf[r][0], kf[r][1]); unpack_bf16x2(kw.y, kf[r][2], kf[r][3]);
        unpack_bf16x2(kw.z, kf[r][4], kf[r][5]); unpack_bf16x2(kw.w, kf[r][6], kf[r][7]);
        unpack_bf16x2(qw.x, qf[0], qf[1]); unpack_bf16x2(qw.y, qf[2], qf[3]);
        unpack_bf16x2(qw.z, qf[4], qf[5]); unpack_bf16x2(qw.w, qf[6], qf[7]);
        const int row = r0 + r;
        *reinterpret_cast<f16x4_t*>(&sm.K[row * KLD + pc_lo]) =
            f16x4_t{(_Float16)kf[r][0], (_Float16)kf[r][1], (_Float16)kf[r][2], (_Float16)kf[r][3]};
        *reinterpret_cast<f16x4_t*>(&sm.K[row * KLD + pc_lo + 8]) =
            f16x4_t{(_Float16)kf[r][4], (_Float16)kf[r][5], (_Float16)kf[r][6], (_Float16)kf[r][7]};
        *reinterpret_cast<f16x4_t*>(&sm.Q[row * KLD + pc_lo]) =
            f16x4_t{(_Float16)qf[0], (_Float16)qf[1], (_Float16)qf[2], (_Float16)qf[3]};
        *reinterpret_cast<f16x4_t*>(&sm.Q[row * KLD + pc_lo + 8]) =
            f16x4_t{(_Float16)qf[4], (_Float16)qf[5], (_Float16)qf[6], (_Float16)qf[7]};
      }
      const int pt = perm16(r0);   // a quad of rows stays contiguous under the permutation
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *reinterpret_cast<f16x4_t*>(&sm.KT[(cc + e) * TLD + pt]) =
            f16x4_t{(_Float16)kf[0][e], (_Float16)kf[1][e], (_Float16)kf[2][e], (_Float16)kf[3][e]};
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): raw rows read, they may be refilled
    if (ch + 1 < n_chunks) issue_kq(ch + 1);
    lds_barrier();

    // ================= P1: A (K K^T, fp32) and P (Q K^T, fp16) tiles, 5 per wave
#pragma unroll
    for (int r = 0; r < 5; ++r) {
      const int task = wave + 4 * r;          // 0..9: K K^T tiles, 10..19: Q K^T tiles
      const bool is_qk = task >= 10;
      const int tile = is_qk ? task - 10 : task;
      const int ti = tile < 1 ? 0 : tile < 3 ? 1 : tile < 6 ? 2 : 3;
      const int tj = tile - (ti * (ti + 1)) / 2;
      const _Float16* X = is_qk ? sm.Q : sm.K;
      f16x8 fa[4], fb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        fa[ks] = ld16(&X[(16 * ti + c16) * KLD + 32 * ks + 8 * g4]);
        fb[ks] = ld16(&sm.K[(16 * tj + c16) * KLD + 32 * ks + 8 * g4]);
      }
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc = mfma16(fa[ks], fb[ks], acc);
      const int cc = 16 * tj + c16;
      const float gc = g_gam[cc];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 16 * ti + 4 * g4 + i;
        const float dec = exp_fast(fminf(g_gam[rr] - gc, 0.f));
        if (!is_qk) sm.A[rr * ALD + cc] = rr > cc ? g_beta[rr] * dec * acc[i] : 0.f;
        else sm.P[rr * TLD + perm16(cc)] = (_Float16)(rr >= cc ? dec * acc[i] : 0.f);
      }
    }
    lds_barrier();

    // ================= P2: diagonal block `wave` of Tm  ||  K S^T, Q S^T, X
    {
      // forward substitution in fp32: column c of (I + A_bb)^-1, bb = wave
      // (the four 16-lane groups compute the same column; all write it)
      const int bb = wave, c = c16;
      const float* Ab = &sm.A[(16 * bb) * ALD + 16 * bb];
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s = (i == c) ? 1.f : 0.f;
#pragma unroll
        for (int j4 = 0; j4 < i; j4 += 4) {
          const f32x4 arow = *reinterpret_cast<const f32x4*>(&Ab[i * ALD + j4]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (j4 + e < i) s = fmaf(-arow[e], x[j4 + e], s);
        }
        x[i] = s;
      }
      const int pc = perm16(16 * bb + c);
#pragma unroll
      for (int i = 0; i < 16; ++i) sm.Tm[(16 * bb + i) * TLD + pc] = (_Float16)x[i];
    }
    f32x16 KS[2], QS[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) { KS[tt] = f32x16{}; QS[tt] = f32x16{}; }
    {
      const _Float16* krow0 = &sm.K[col * KLD + 8 * h];
      const _Float16* qrow0 = &sm.Q[col * KLD + 8 * h];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const f16x8 sb = pack8(Sacc[j], s);
          const int kc = 32 * j + 16 * s;
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            KS[tt] = mfma32(ld16(krow0 + 32 * tt * KLD + kc), sb, KS[tt]);
            QS[tt] = mfma32(ld16(qrow0 + 32 * tt * KLD + kc), sb, QS[tt]);
          }
        }
      }
    }
    // X = beta (V - e^gam K S^T) in place of KS; e^gam Q S^T in place of QS
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int t4 = 32 * tt + 8 * g + 4 * h;     // rows of elements 4g..4g+3
        const f32x4 eg = *reinterpret_cast<const f32x4*>(&g_eg[t4]);
        const f32x4 bt = *reinterpret_cast<const f32x4*>(&g_beta[t4]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 4 * g + r;
          KS[tt][i] = bt[r] * (bf16_bits_to_f32(sV[(t4 + r) * D + vrow]) - eg[r] * KS[tt][i]);
          QS[tt][i] *= eg[r];
        }
      }
    }
    lds_barrier();

    // ================= P3: block merges of Tm (wave 0); gates of chunk ch+1 (wave 1);
    // V of chunk ch+1 (every wave has read V of chunk ch)
    if (ch + 1 < n_chunks) {
      if (wave == 1) gates_chunk(ch + 1);   // its loads were issued before the K/Q DMA
      issue_v(ch + 1);
    }
    if (wave == 0) {
#pragma unroll
      for (int a0 = 0; a0 < 64; a0 += 32) {
        // 16-merges inside the diagonal 32-blocks: T21 = -T22 (A21 T11)
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(&sm.A[(a0 + 16 + c16) * ALD + a0 + 4 * g4]);
        const f16x4_t fa = {(_Float16)a4[0], (_Float16)a4[1], (_Float16)a4[2], (_Float16)a4[3]};
        f16x4_t fb;
        const int pcb = perm16(a0 + c16);
#pragma unroll
        for (int e = 0; e < 4; ++e) fb[e] = sm.Tm[(a0 + 4 * g4 + e) * TLD + pcb];
        const f32x4 y = mfma16k16(fa, fb, f32x4{0.f, 0.f, 0.f, 0.f});
        const f16x4_t ft =
            *reinterpret_cast<const f16x4_t*>(&sm.Tm[(a0 + 16 + c16) * TLD + perm16(a0 + 16 + 4 * g4)]);
        const f16x4_t fy = {(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
        const f32x4 t21 = mfma16k16(ft, fy, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.Tm[(a0 + 16 + 4 * g4 + i) * TLD + pcb] = (_Float16)(-t21[i]);
      }
      // 32-merge: T_ba = -T_b (A_ba T_a), a = rows/cols 0..31, b = 32..63
      f32x16 y = f32x16{};
      const int pcol = perm16(col);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        f16x8 fb;
#pragma unroll
        for (int e = 0; e < 8; ++e) fb[e] = sm.Tm[(16 * s + 8 * h + e) * TLD + pcol];
        y = mfma32(ld_f32x8_as_f16(&sm.A[(32 + col) * ALD + 16 * s + 8 * h]), fb, y);
      }
      f32x16 tba = f32x16{};
#pragma unroll
      for (int s = 0; s < 2; ++s)
        tba = mfma32(ld16(&sm.Tm[(32 + col) * TLD + 32 + 16 * s + 8 * h]), pack8(y, s), tba);
#pragma unroll
      for (int i = 0; i < 16; ++i) sm.Tm[(32 + acc_row(i, h)) * TLD + pcol] = (_Float16)(-tba[i]);
    }
    lds_barrier();

    // ================= P4: Vn = Tm X, O = scale (e^gam Q S^T + P Vn), state update
    {
      f16x8 Xb[2][2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) { Xb[tt][0] = pack8(KS[tt], 0); Xb[tt][1] = pack8(KS[tt], 1); }
      f16x8 Vnb[2][2], Vdb[2][2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        f32x16 vn = f32x16{};
        const _Float16* trow = &sm.Tm[(32 * tt + col) * TLD + 8 * h];
#pragma unroll
        for (int tp = 0; tp <= tt; ++tp) {
#pragma unroll
          for (int s = 0; s < 2; ++s) vn = mfma32(ld16(trow + 32 * tp + 16 * s), Xb[tp][s], vn);
        }
        Vnb[tt][0] = pack8(vn, 0);
        Vnb[tt][1] = pack8(vn, 1);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 ed = *reinterpret_cast<const f32x4*>(&g_ed[32 * tt + 8 * g + 4 * h]);
#pragma unroll
          for (int r = 0; r < 4; ++r) vn[4 * g + r] *= ed[r];
        }
        Vdb[tt][0] = pack8(vn, 0);
        Vdb[tt][1] = pack8(vn, 1);
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const _Float16* prow = &sm.P[(32 * tt + col) * TLD + 8 * h];
#pragma unroll
        for (int tp = 0; tp <= tt; ++tp) {
#pragma unroll
          for (int s = 0; s < 2; ++s) QS[tt] = mfma32(ld16(prow + 32 * tp + 16 * s), Vnb[tp][s], QS[tt]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
          opack[tt][i] = pack_bf16x2(scale * QS[tt][2 * i], scale * QS[tt][2 * i + 1]);
      }
      o_t0 = t0;
      const float egL = g_eg[L - 1];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Sacc[j] *= egL;
        const _Float16* ktrow = &sm.KT[(32 * j + col) * TLD + 8 * h];
#pragma unroll
        for (int tp = 0; tp < 2; ++tp) {
#pragma unroll
          for (int s = 0; s < 2; ++s) Sacc[j] = mfma32(ld16(ktrow + 32 * tp + 16 * s), Vdb[tp][s], Sacc[j]);
        }
      }
    }
    lds_barrier();
  }

  // ---- output of the last chunk (rows past its end are not written)
  if (n_chunks > 0) {
    const int L = len - (n_chunks - 1) * C;
    const uint32_t loff = uint32_t(vrow) + uint32_t(4 * h) * uint32_t(v_stride);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 4 * g + r;
          uint16_t* rowp = out + size_t(o_t0 + 32 * tt + 8 * g + r) * v_stride + size_t(hv) * D;
          if (32 * tt + acc_row(i, h) < L) rowp[loff] = uint16_t(opack[tt][i >> 1] >> (16 * (i & 1)));
        }
      }
    }
  }

  // ---- final state
  float* dst = ht + state_off;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *reinterpret_cast<f32x4*>(dst + 32 * j + 8 * g + 4 * h) =
          f32x4{Sacc[j][4 * g + 0], Sacc[j][4 * g + 1], Sacc[j][4 * g + 2], Sacc[j][4 * g + 3]};
    }
  }
}

int check_prefill_args(const void* q, const void* k, const void* v, const void* A_log,
                       const void* a, const void* dt_bias, const void* b, const void* cu,
                       const void* out, const void* final_state, int N, int T, int HQ, int HV) {
  if (!q || !k || !v || !A_log || !a || !dt_bias || !b || !cu || !out || !final_state)
    return GDN_ERR_NULL;
  if (N < 0 || T < 0 || HQ <= 0 || HV <= 0 || HV % HQ != 0) return GDN_ERR_SHAPE;
  return GDN_OK;
}

}  // namespace

extern "C" size_t gdn_prefill_workspace_bytes(int, int, int, int) { return 0; }

extern "C" int gdn_prefill_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const float* state, const float* A_log, const uint16_t* a,
                               const float* dt_bias, const uint16_t* b, const void* cu_seqlens,
                               int cu_is_int32, int N, int T, int HQ, int HV, float scale,
                               uint16_t* out, float* final_state, void* workspace,
                               size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  const int rc = check_prefill_args(q, k, v, A_log, a, dt_bias, b, cu_seqlens, out, final_state,
                                    N, T, HQ, HV);
  if (rc != GDN_OK) return rc;
  if (N == 0) return GDN_OK;
  const dim3 grid(unsigned(N) * unsigned(HV));
  const dim3 block(kThreads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (cu_is_int32) {
    hipLaunchKernelGGL(gdn_prefill_chain_kernel<int32_t>, grid, block, 0, st, q, k, v, state,
                       A_log, a, dt_bias, b, static_cast<const int32_t*>(cu_seqlens), T, HQ, HV,
                       scale, out, final_state);
  } else {
    hipLaunchKernelGGL(gdn_prefill_chain_kernel<int64_t>, grid, block, 0, st, q, k, v, state,
                       A_log, a, dt_bias, b, static_cast<const int64_t*>(cu_seqlens), T, HQ, HV,
                       scale, out, final_state);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? GDN_OK : -int(err);
}
