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
//   Tm  = (I + A)^-1                                       (fp32, blocked 16x16)
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
constexpr int KLD = D + 4;    // sK / sQ row stride (halves): 264 B rows
constexpr int TLD = C + 4;    // sKT / sTm / sP row stride (halves): 136 B rows
constexpr int FLD = C + 1;    // sA / sTF row stride (floats)
constexpr int kThreads = 256;

struct __align__(16) Smem {
  _Float16 K[C * KLD];        // K chunk, [t][k]
  _Float16 Q[C * KLD];        // Q chunk, [t][k]
  _Float16 KT[D * TLD];       // K chunk transposed, [k][t]
  _Float16 Tm[C * TLD];       // (I + A)^-1, [t][t']
  _Float16 P[C * TLD];        // decayed causal Q K^T, [t][t']
  float A[C * FLD];           // beta-scaled decayed strict K K^T (fp32)
  float TF[C * FLD];          // (I + A)^-1 in fp32
  float Y[3 * 16 * 17];       // per-wave 16x16 scratch of the inverse
  float gam[C];               // chunk-local cumsum of the log-decay
  float beta[C];
  float eg[C];                // e^{gam_t}
  float ed[C];                // e^{gam_{L-1} - gam_t}
};

__device__ __forceinline__ f16x8 ld_frag_split(const _Float16* row, int col) {
  // halves [col, col+4) and [col+8, col+12) of one row (two 8-byte LDS reads)
  const f16x4 lo = *reinterpret_cast<const f16x4*>(row + col);
  const f16x4 hi = *reinterpret_cast<const f16x4*>(row + col + 8);
  return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ f16x8 ld_frag_contig(const _Float16* row, int col) {
  // halves [col, col+8) of one row (two 8-byte LDS reads)
  const f16x4 lo = *reinterpret_cast<const f16x4*>(row + col);
  const f16x4 hi = *reinterpret_cast<const f16x4*>(row + col + 4);
  return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
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

// Row t of an accumulator tile element i for lane half h (32x32 layout).
__device__ __forceinline__ int acc_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

template <typename CuT>
__global__ __launch_bounds__(kThreads, 1) void gdn_prefill_chain_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ h0,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    const CuT* __restrict__ cu_seqlens, int T, int HQ, int HV, float scale,
    uint16_t* __restrict__ out, float* __restrict__ ht) {
  __shared__ Smem sm;

  const int n = blockIdx.x / HV;
  const int hv = blockIdx.x - n * HV;
  const int hq = hv / (HV / HQ);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int h = lane >> 5;        // lane half (32x32 MFMA layouts)
  const int col = lane & 31;
  const int vrow = 32 * wave + col;   // state row v owned by this lane

  long long bos_l = (long long)cu_seqlens[n];
  long long eos_l = (long long)cu_seqlens[n + 1];
  bos_l = bos_l < 0 ? 0 : (bos_l > T ? T : bos_l);
  eos_l = eos_l < bos_l ? bos_l : (eos_l > T ? T : eos_l);
  const int bos = int(bos_l);
  const int len = int(eos_l - bos_l);

  const float a_log_exp = expf(A_log[hv]);
  const float dtb = dt_bias[hv];

  // Upper 16x16 tiles inside the diagonal 32x32 blocks of Tm / P are read by
  // the 32x32 products and must be zero; they are never written afterwards.
  for (int e = tid; e < 2 * 16 * 16; e += kThreads) {
    const int blk = e >> 8, r = (e >> 4) & 15, c = e & 15;
    const int R = 32 * blk + r, Cc = 32 * blk + 16 + c;
    sm.Tm[R * TLD + Cc] = (_Float16)0.f;
    sm.P[R * TLD + Cc] = (_Float16)0.f;
  }

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

  const size_t qk_stride = size_t(HQ) * D;   // elements per token in q / k
  const size_t v_stride = size_t(HV) * D;    // elements per token in v / out
  const int n_chunks = (len + C - 1) / C;

  for (int ch = 0; ch < n_chunks; ++ch) {
    const int t0 = bos + ch * C;
    const int L = min(C, len - ch * C);

    // ---------------- phase 0: K, Q -> LDS (fp16), K^T, gates
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int seg = tid + kThreads * r;     // 1024 segments of 8 halves
      const int row = seg >> 4;
      const int c8 = (seg & 15) * 8;
      uint4 kw = make_uint4(0, 0, 0, 0), qw = make_uint4(0, 0, 0, 0);
      if (row < L) {
        const size_t off = size_t(t0 + row) * qk_stride + size_t(hq) * D + c8;
        kw = *reinterpret_cast<const uint4*>(k + off);
        qw = *reinterpret_cast<const uint4*>(q + off);
      }
      float kf[8], qf[8];
      unpack_bf16x2(kw.x, kf[0], kf[1]); unpack_bf16x2(kw.y, kf[2], kf[3]);
      unpack_bf16x2(kw.z, kf[4], kf[5]); unpack_bf16x2(kw.w, kf[6], kf[7]);
      unpack_bf16x2(qw.x, qf[0], qf[1]); unpack_bf16x2(qw.y, qf[2], qf[3]);
      unpack_bf16x2(qw.z, qf[4], qf[5]); unpack_bf16x2(qw.w, qf[6], qf[7]);
      f16x4 k0, k1, q0, q1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        k0[e] = (_Float16)kf[e]; k1[e] = (_Float16)kf[4 + e];
        q0[e] = (_Float16)qf[e]; q1[e] = (_Float16)qf[4 + e];
      }
      *reinterpret_cast<f16x4*>(&sm.K[row * KLD + c8]) = k0;
      *reinterpret_cast<f16x4*>(&sm.K[row * KLD + c8 + 4]) = k1;
      *reinterpret_cast<f16x4*>(&sm.Q[row * KLD + c8]) = q0;
      *reinterpret_cast<f16x4*>(&sm.Q[row * KLD + c8 + 4]) = q1;
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.KT[(c8 + e) * TLD + row] = (_Float16)kf[e];
    }
    if (wave == 0) {
      const int t = lane;
      float ld = 0.f, bt = 0.f;
      if (t < L) {
        const size_t gi = size_t(t0 + t) * HV + hv;
        const float x = bf16_bits_to_f32(a[gi]) + dtb;
        ld = -a_log_exp * softplus_stable(x);
        bt = sigmoidf_(bf16_bits_to_f32(b[gi]));
      }
      // inclusive scan over the 64 lanes
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(ld, off, 64);
        if (lane >= off) ld += y;
      }
      const float gl = __shfl(ld, L - 1, 64);
      sm.gam[t] = ld;
      sm.beta[t] = bt;
      sm.eg[t] = expf(ld);
      sm.ed[t] = expf(gl - ld);
    }
    __syncthreads();

    // ---------------- phase 1: A (strict, beta-scaled) and P (inclusive) tiles
    {
      const int g4 = lane >> 4;    // 16x16 layouts: lane group
      const int c16 = lane & 15;
#pragma unroll
      for (int r = 0; r < 5; ++r) {
        const int task = wave + 4 * r;          // 0..9: K K^T tiles, 10..19: Q K^T tiles
        const bool is_qk = task >= 10;
        const int tile = is_qk ? task - 10 : task;
        // lower tiles (ti >= tj) of the 4x4 grid of 16x16 tiles
        const int ti = tile < 1 ? 0 : tile < 3 ? 1 : tile < 6 ? 2 : 3;
        const int tj = tile - (ti * (ti + 1)) / 2;
        const _Float16* X = is_qk ? sm.Q : sm.K;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const f16x8 fa = ld_frag_contig(&X[(16 * ti + c16) * KLD], 32 * ks + 8 * g4);
          const f16x8 fb = ld_frag_contig(&sm.K[(16 * tj + c16) * KLD], 32 * ks + 8 * g4);
          acc = mfma16(fa, fb, acc);
        }
        const int cc = 16 * tj + c16;
        const float gc = sm.gam[cc];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = 16 * ti + 4 * g4 + i;
          const float dec = expf(fminf(sm.gam[rr] - gc, 0.f));
          if (!is_qk) {
            sm.A[rr * FLD + cc] = rr > cc ? sm.beta[rr] * dec * acc[i] : 0.f;
          } else {
            sm.P[rr * TLD + cc] = (_Float16)(rr >= cc ? dec * acc[i] : 0.f);
          }
        }
      }
    }
    __syncthreads();

    // ---------------- phase 2: Tm = (I + A)^-1, blocked 16x16, fp32
    if (wave == 0) {
      // diagonal blocks by forward substitution; lane = (block, column)
      const int bb = lane >> 4, c = lane & 15;
      const float* Ab = &sm.A[(16 * bb) * FLD + 16 * bb];
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s = (i == c) ? 1.f : 0.f;
#pragma unroll
        for (int j = 0; j < i; ++j) s = fmaf(-Ab[i * FLD + j], x[j], s);
        x[i] = s;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sm.TF[(16 * bb + i) * FLD + 16 * bb + c] = x[i];
    }
    __syncthreads();
    {
      // off-diagonal blocks, level by level:  T_ij = -T_ii * sum_{j<=m<i} A_im T_mj
      const int g4 = lane >> 4, c = lane & 15;
      float* Yw = &sm.Y[(wave < 3 ? wave : 0) * 16 * 17];
#pragma unroll 1
      for (int lvl = 1; lvl <= 3; ++lvl) {
        const bool active = wave < 4 - lvl;
        const int bj = wave, bi = wave + lvl;
        if (active) {
          float y[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rr = 4 * g4 + i;
            float s = 0.f;
            for (int bm = bj; bm < bi; ++bm) {
              const float* Arow = &sm.A[(16 * bi + rr) * FLD + 16 * bm];
              const float* Tcol = &sm.TF[(16 * bm) * FLD + 16 * bj + c];
#pragma unroll
              for (int m = 0; m < 16; ++m) s = fmaf(Arow[m], Tcol[m * FLD], s);
            }
            y[i] = s;
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) Yw[(4 * g4 + i) * 17 + c] = y[i];
        }
        __syncthreads();
        if (active) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rr = 4 * g4 + i;
            const float* Trow = &sm.TF[(16 * bi + rr) * FLD + 16 * bi];
            float s = 0.f;
#pragma unroll
            for (int m = 0; m < 16; ++m) s = fmaf(Trow[m], Yw[m * 17 + c], s);
            sm.TF[(16 * bi + rr) * FLD + 16 * bj + c] = -s;
          }
        }
        __syncthreads();
      }
    }
    for (int e = tid; e < C * C; e += kThreads) {
      const int rr = e >> 6, cc = e & 63;
      // the upper tiles of the diagonal 32-blocks stay zero from the prologue
      if (rr >= cc) sm.Tm[rr * TLD + cc] = (_Float16)sm.TF[rr * FLD + cc];
      else if ((rr >> 5) == (cc >> 5) && ((rr >> 4) & 1) == ((cc >> 4) & 1))
        sm.Tm[rr * TLD + cc] = (_Float16)0.f;
    }
    __syncthreads();

    // ---------------- phase 3: the state-dependent chain for rows [32w, 32w+32)
    {
      // V slice in accumulator layout (issued early)
      float Vv[2][16];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int t = 32 * tt + acc_row(i, h);
          Vv[tt][i] = t < L ? bf16_bits_to_f32(v[size_t(t0 + t) * v_stride + size_t(hv) * D + vrow]) : 0.f;
        }
      }

      f16x8 Sb[4][2];
#pragma unroll
      for (int j = 0; j < 4; ++j) { Sb[j][0] = pack8(Sacc[j], 0); Sb[j][1] = pack8(Sacc[j], 1); }

      f32x16 KS[2], QS[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        KS[tt] = f32x16{};
        QS[tt] = f32x16{};
        const _Float16* krow = &sm.K[(32 * tt + col) * KLD];
        const _Float16* qrow = &sm.Q[(32 * tt + col) * KLD];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const int kc = 32 * j + 16 * s + 4 * h;
            KS[tt] = mfma32(ld_frag_split(krow, kc), Sb[j][s], KS[tt]);
            QS[tt] = mfma32(ld_frag_split(qrow, kc), Sb[j][s], QS[tt]);
          }
        }
      }

      // X = beta (V - e^gam K S^T)   (reuses KS)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int t = 32 * tt + acc_row(i, h);
          KS[tt][i] = sm.beta[t] * (Vv[tt][i] - sm.eg[t] * KS[tt][i]);
        }
      }
      f16x8 Xb[2][2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) { Xb[tt][0] = pack8(KS[tt], 0); Xb[tt][1] = pack8(KS[tt], 1); }

      // Vn = Tm X  (Tm lower triangular in 32-blocks)
      f32x16 Vn[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const _Float16* trow = &sm.Tm[(32 * tt + col) * TLD];
#pragma unroll
        for (int tp = 0; tp <= tt; ++tp) {
#pragma unroll
          for (int s = 0; s < 2; ++s)
            Vn[tt] = mfma32(ld_frag_split(trow, 32 * tp + 16 * s + 4 * h), Xb[tp][s], Vn[tt]);
        }
      }
      f16x8 Vnb[2][2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) { Vnb[tt][0] = pack8(Vn[tt], 0); Vnb[tt][1] = pack8(Vn[tt], 1); }

      // O = scale (e^gam Q S^T + P Vn)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) QS[tt][i] *= sm.eg[32 * tt + acc_row(i, h)];
        const _Float16* prow = &sm.P[(32 * tt + col) * TLD];
#pragma unroll
        for (int tp = 0; tp <= tt; ++tp) {
#pragma unroll
          for (int s = 0; s < 2; ++s)
            QS[tt] = mfma32(ld_frag_split(prow, 32 * tp + 16 * s + 4 * h), Vnb[tp][s], QS[tt]);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int t = 32 * tt + acc_row(i, h);
          if (t < L)
            out[size_t(t0 + t) * v_stride + size_t(hv) * D + vrow] = f32_to_bf16_bits(scale * QS[tt][i]);
        }
      }

      // S <- e^{gam_L} S + (e^{gam_L - gam} Vn)^T K
      f16x8 Vdb[2][2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) Vn[tt][i] *= sm.ed[32 * tt + acc_row(i, h)];
        Vdb[tt][0] = pack8(Vn[tt], 0);
        Vdb[tt][1] = pack8(Vn[tt], 1);
      }
      const float egL = sm.eg[L - 1];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Sacc[j] *= egL;
        const _Float16* ktrow = &sm.KT[(32 * j + col) * TLD];
#pragma unroll
        for (int tp = 0; tp < 2; ++tp) {
#pragma unroll
          for (int s = 0; s < 2; ++s)
            Sacc[j] = mfma32(ld_frag_split(ktrow, 32 * tp + 16 * s + 4 * h), Vdb[tp][s], Sacc[j]);
        }
      }
    }
    __syncthreads();
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
