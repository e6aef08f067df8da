// GDN chunked varlen prefill for batches with fewer (sequence, v-head) chains
// than the GPU has CUs (gfx950 / CDNA4, wave64, MFMA).  Two launches:
//
//  1. gdn_prefill_prep_kernel: one workgroup per (chunk, v-head), every chunk
//     of every sequence at once.  It forms what of a chunk does not depend on
//     the state -- the gates, A = tril_strict(beta_i e^{gam_i-gam_j} K K^T),
//     the diagonal 32-row blocks of Tm = (I + A)^-1, -A_ba (the lower-left
//     32x32 block of A) and P = scale tril_incl(e^{gam_i-gam_j} Q K^T) -- and
//     writes it to the workspace as ready MFMA operand fragments.  This is
//     the work of the reference's chunk_scaled_dot_kkt_fwd and
//     recompute_w_u_fwd (gdn_prefill_qk4_v8_d128_k_last/solution/triton/
//     kernel.py:473-559, 617-796, gating :1706-1722) run over all chunks in
//     parallel, as the reference launches them (grids over chunks, :544,
//     :1005), but stopping before W and U.
//  2. gdn_prefill_slice_kernel: one workgroup per (sequence, v-head, slice of
//     R state rows).  The rows of the state evolve independently -- with
//     X = beta (V - e^gam K S^T) and Vn = Tm X every product that touches S,
//     X, Vn or O is row-separable in v -- so a chain splits over 128 / R
//     workgroups that never exchange data (the reference splits its
//     recurrence the same way, grid (V / BV, N H), kernel.py:1369).  Each
//     workgroup walks the chunks of its sequence in order with its rows of
//     S in MFMA accumulators: K S^T, X, Vn = Tm X (two-level, as in the
//     fused kernel), O = scale e^gam Q S^T + P Vn, S <- e^{gam_L} S + K^T Vd.
//
// Arithmetic and operand precisions are those of the fused chain kernel
// (gdn_prefill.hip): bf16 MFMA for A and P from the exact bf16 rows, fp16
// operands on the state path, bf16 S for Q S^T, fp32 accumulation.

#include <algorithm>
#include <mutex>

#include "gdn_prefill_common.h"
#include "gdn_prefill_split.h"
#include "../../include/gdn_hip.h"

namespace {

using namespace gdn;

// ---------------------------------------------------------------------------
// Workspace record of one (chunk, v-head), 14 080 bytes.  An operand
// fragment is 1 KB: lane l's 16 bytes at 16 l, exactly the register image a
// 16x16x32 MFMA operand read gives lane l, so readers copy it whole and read
// it back with one conflict-free 16-byte LDS read per lane.
constexpr int kFrag = 1024;
constexpr int BL_TM = 0;               // 4 fragments: T_a rows 0-15, 16-31; T_b rows 32-47, 48-63
constexpr int BL_AB = 4 * kFrag;       // 2 fragments: -A_ba rows 32-47, 48-63
constexpr int BL_P = 6 * kFrag;        // 6 fragments: P (token block, column block) 00 10 20 21 30 31
constexpr int BL_G = 12 * kFrag;       // gate data, GSZ floats (layout of the G_* offsets)
constexpr int BL_N = BL_G + 4 * GSZ;   // GDN_QK_L2NORM: row factors of K (64 floats), then of Q
constexpr int kBlob = BL_N + 4 * 2 * C;
static_assert(kBlob % 256 == 0, "records stay 256-byte aligned");
// fp16 K rows of one (chunk, qk-head) as the chain reads them in LDS: [t][p32(k)]
// with KCLD-element rows (the padding is never read), rows past the chunk end 0.
constexpr int kKcBytes = C * KCLD * 2;
static_assert(kKcBytes % kFrag == 0, "whole 1 KB copies");
constexpr int kKcCopies = kKcBytes / kFrag;
// gate data and L2-norm factors of a record, staged in LDS by the state slices
constexpr int kGateBytes = kBlob - BL_G;
constexpr int kGateCopies = (kGateBytes + kFrag - 1) / kFrag;

constexpr int kPrepThreads = 256;
// Batches of up to this many sequences have their slice workgroups ordered
// longest sequence first (the preparation launch ranks the sequences).
constexpr int kMaxOrdered = 4096;

// The workspace: the (chunk, v-head) records, the fp16 K images of every
// (chunk, qk-head), then the sequence order of the slice launch (N ints).
__host__ __device__ inline size_t order_offset(int n_slots, int HQ, int HV) {
  return size_t(n_slots) * (size_t(HV) * size_t(kBlob) + size_t(HQ) * size_t(kKcBytes));
}

// ---------------------------------------------------------------------------
// Time splits ("seams") of long chains.  With workgroups to spare (few chains
// on many CUs) a sequence of Lc chunks is cut at sp = ceil(Lc / 2): its head
// [0, sp) runs as usual from the initial state; its tail [sp, Lc) runs at the
// same time twice, from a zero state (giving the tail's outputs O0 and final
// state S0) and as the transition chain: the same recurrence with v = 0 from
// the identity, whose "state" X_c is the product of the tail's per-chunk
// transitions M (S_{c+1} = S_c M_c + B_c, M independent of v) and whose
// outputs OX_c = G_c X_c^T are the outputs' linear part.  With S_sp the head's
// final state, the true tail outputs are O0_c + OX_c S_sp^T and the final
// state S_sp X + S0; gdn_prefill_seam_kernel adds those terms.
//
// The plan is made on the device from the sequences ranked by length
// (order[]): seams go to the j longest sequences, j <= the workgroups left
// idle allow, choosing j by a chunk-period model (a split halves the longest
// chain; the seam pass costs about kSeamCostChunks chunk periods).
constexpr int kSeamMaxChains = 64;    // (sequence, v-head) chains up to which seams are considered
constexpr int kSeamMinChunks = 8;     // shortest chain split
constexpr int kSeamCostChunks = 5;    // seam pass, in chunk periods of a slice

__host__ __device__ inline int seam_split_chunk(int chunks) { return (chunks + 1) / 2; }

// XCD of the first seam group: the groups continue the rotation where the
// chains' last, partial row of units left XCDs idle (an even row fills XCDs
// 0 .. r-1, an odd one 8-r .. 7).
__host__ __device__ inline int seam_xcd_offset(int n_units) {
  const int r = n_units & 7;
  return (r == 0 || (((n_units - 1) >> 3) & 1)) ? 0 : r;
}

// Seams the grid has room for (host and device).  Every workgroup of the
// slice launch holds a CU, and the dispatcher keeps each workgroup on the
// XCD its id names (id mod 8), so the count is per XCD: each chain unit puts
// G * slices workgroups on its XCD, each seam 2 HQ groups of G * slices (the
// tails, the transition chains), and a seam is admitted only while every XCD
// keeps at most cus / 8 of them: a tail that waited for a CU would run after
// the head it is meant to run beside.
__host__ __device__ inline int seam_room(int N, int HQ, int HV, int slices, int cus) {
  const long long chains = (long long)N * HV;
  if (HQ <= 0 || chains <= 0 || chains > kSeamMaxChains || cus <= 0) return 0;
  const int per_xcd = cus / 8, units = N * HQ, group = (HV / HQ) * slices;
  int load[8] = {};
  for (int su = 0; su < units; ++su) {
    const int jx = su >> 3, x = su & 7;
    load[(jx & 1) ? 7 - x : x] += group;
  }
  int worst = 0;
  for (int x = 0; x < 8; ++x) worst = load[x] > worst ? load[x] : worst;
  if (worst > per_xcd) return 0;
  const int off = seam_xcd_offset(units);
  const int k_max = N < kMaxSeams ? N : kMaxSeams;
  int k = 0;
  for (int kk = 1; kk <= k_max; ++kk) {
    bool fits = true;
    for (int gi = 2 * (kk - 1) * HQ; gi < 2 * kk * HQ; ++gi) {
      int& l = load[(gi + off) & 7];
      l += group;
      fits = fits && l <= per_xcd;
    }
    if (!fits) break;
    k = kk;
  }
  return k;
}

// The seam region of the split path follows the order[] ints; its slots:
// min(N, kMaxSeams), its OX rows seam_ox_rows(N, T).  The slice launch writes
// the plan (slots past the seam count get sequence -1).
__host__ __device__ inline size_t seam_plan_offset(int n_slots, int N, int HQ, int HV) {
  return order_offset(n_slots, HQ, HV) + (size_t(N) * sizeof(int) + 255) / 256 * 256;
}
__host__ __device__ inline int seam_slots(int N) { return N < kMaxSeams ? N : kMaxSeams; }
__host__ __device__ inline int seam_ox_rows(int N, int T) { return T / 2 + C * seam_slots(N); }
__host__ __device__ inline size_t seam_bytes(int N, int T, int HV) {
  if ((long long)N * HV > kSeamMaxChains) return kSeamPlanBytes;
  return seam_region_bytes(seam_slots(N), HV, seam_ox_rows(N, T));
}

// The seams of a launch, identical in every workgroup and in the seam pass:
// their count; the split chunk of seam j is seam_split_chunk of the chunk
// count of sequence order[j].  Chunk counts are clamped as the chains clamp
// them.  Wave-uniform.
// chunks_of(r): chunk count of the r-th longest sequence.  Returns the seam
// count and sets *span to the modelled finish in chunk periods of a slice
// (the longest chain's chunks without seams).  Host and device.
template <typename ChunksOf>
__host__ __device__ inline int seam_choice(ChunksOf chunks_of, int N, int room, int* span) {
  const int l0 = N > 0 ? chunks_of(0) : 0;
  int best = l0, best_k = 0;
  for (int kk = 1; kk <= room; ++kk) {
    if (chunks_of(kk - 1) < kSeamMinChunks) break;
    const int rest = kk < N ? chunks_of(kk) : 0;
    const int sp = seam_split_chunk(l0);
    const int span_k = (sp > rest ? sp : rest) + kSeamCostChunks;
    if (span_k < best) {
      best = span_k;
      best_k = kk;
    }
  }
  *span = best;
  return best_k;
}

template <typename CuT>
__device__ int seam_count(const CuT* cu, const int* order, int N, int T, int room) {
  if (room <= 0) return 0;
  auto chunks_of = [&](int r) {
    const int nn = order[r];
    int bb, ll;
    seq_bounds(cu, nn, T, bb, ll);
    return (ll + C - 1) / C;
  };
  int span;
  return seam_choice(chunks_of, N, room, &span);
}

// OX rows of the seams before seam j (their tail tokens).  OX holds
// seam_ox_rows(N, T) rows; writers drop rows past it (ranges that overlap
// can ask for more).
template <typename CuT>
__device__ int seam_rows_before(const CuT* cu, const int* order, int T, int j) {
  int row = 0;
  for (int jj = 0; jj < j; ++jj) {
    int bb, ll;
    seq_bounds(cu, order[jj], T, bb, ll);
    row += max(0, ll - C * seam_split_chunk((ll + C - 1) / C));
  }
  return row;
}

// HBM -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): from
// base + off (base uniform, off a 32-bit lane offset) to LDS byte address
// lds + 16 l for lane l (lds uniform).  Issued from asm so that the compiler
// places no waits for it; consumers wait with explicit vmcnt counts and a
// barrier.  The LDS address is a fixed M0 operand, written by the compiler.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// ---------------------------------------------------------------------------
// Preparation of one chunk of one v-head.  Four waves:
//   copies   raw K and Q rows (bf16) of the chunk into LDS, swizzled;
//   wave 0   gates (softplus, sigmoid, chunk-local cumsum by a DPP scan);
//   all      (option) L2-norm factors of the 128 rows; 20 A / P tiles;
//   wave 0   the four diagonal 16x16 blocks of Tm by forward substitution;
//   waves 2-3  the two 16-row merges inside the diagonal 32-row blocks;
//   all      the operand fragments to the workspace, and (first v-head of
//            each qk-head) the fp16 K rows in the chain's LDS layout.
// Rows past the chunk end are copies of its last row with beta = 0 and a
// zero log-decay, so their A rows vanish and their Tm rows are unit rows.
template <typename CuT, bool kL2>
__global__ __launch_bounds__(kPrepThreads) void gdn_prefill_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    const CuT* __restrict__ cu_seqlens, int N, int T, int HQ, int HV, float scale,
    char* __restrict__ blob, int n_slots) {
  __shared__ __align__(16) uint16_t rk[C * D];
  __shared__ __align__(16) uint16_t rq[C * D];
  __shared__ __align__(16) float sA[C * ALD];
  __shared__ __align__(16) _Float16 sTm[C * TLD];
  __shared__ __align__(16) _Float16 sP[C * TLD];
  __shared__ __align__(16) _Float16 sAba[(C / 2) * BLD];
  __shared__ __align__(16) float gd[GSZ];
  __shared__ __align__(16) float nrm[2 * C];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const size_t qk_stride = size_t(HQ) * D;
  const int heads_per_qk = HV / HQ;

  // order[r] = the sequence of rank r by descending length (ties: lower index
  // first), read by the slice launch to start the longest chains first.
  {
    int* order = reinterpret_cast<int*>(blob + order_offset(n_slots, HQ, HV));
    for (int n = blockIdx.x * kPrepThreads + tid; n < N; n += gridDim.x * kPrepThreads) {
      int rank = n;
      if (N <= kMaxOrdered) {
        int b0, l0;
        seq_bounds(cu_seqlens, n, T, b0, l0);
        rank = 0;
        for (int m = 0; m < N; ++m) {
          int b1, l1;
          seq_bounds(cu_seqlens, m, T, b1, l1);
          rank += (l1 > l0 || (l1 == l0 && m < n)) ? 1 : 0;
        }
      }
      order[rank] = n;
    }
  }

  // The upper 16x16 tiles inside the diagonal 32x32 blocks of Tm and P are
  // part of the fragments and must be zero; nothing else writes them.
  for (int e = tid; e < 2 * 16 * 16; e += kPrepThreads) {
    const int blk = e >> 8, r = (e >> 4) & 15, cc = e & 15;
    const int R0 = 32 * blk + r, pc = p32(32 * blk + 16 + cc);
    sTm[R0 * TLD + pc] = (_Float16)0.f;
    sP[R0 * TLD + pc] = (_Float16)0.f;
  }

  // Persistent workgroups: unit u = (slot u / HV, v-head u % HV), this
  // workgroup taking u = blockIdx.x, + gridDim.x, ...  The raw K / Q rows and
  // the gate inputs of the next unit are loaded into registers while the
  // current one is processed.  Slots past the last chunk end the walk (a
  // later unit has a later or equal slot).
  const int n_units = n_slots * HV;
  struct Unit { int slot, hv, t0, L; };
  auto locate = [&](int u, Unit& x) {
    x.slot = u / HV;
    x.hv = u - x.slot * HV;
    int n, ci;
    locate_chunk(cu_seqlens, N, T, x.slot, lane, n, ci);
    if (n < 0) return false;
    int bos, len;
    seq_bounds(cu_seqlens, n, T, bos, len);
    x.t0 = bos + ci * C;
    x.L = min(C, len - ci * C);
    return true;
  };
  constexpr int kRowLoads = (C * D / 8) / kPrepThreads;
  static_assert(kRowLoads == 4, "four 16-byte row pieces per thread");
  uint4 pk0, pk1, pk2, pk3, pq0, pq1, pq2, pq3;
  uint16_t pa = 0, pb = 0;
  float pdt = 0.f, pal = 0.f;
  auto fetch = [&](const Unit& x) {
    const int hq_ = x.hv / heads_per_qk;
    auto src = [&](int j) {
      const int item = tid + kPrepThreads * j;
      const int row = item >> 4, pc = item & 15;
      return size_t(x.t0 + min(row, x.L - 1)) * qk_stride + size_t(hq_) * D + 8 * pc;
    };
    pk0 = *reinterpret_cast<const uint4*>(k + src(0));
    pq0 = *reinterpret_cast<const uint4*>(q + src(0));
    pk1 = *reinterpret_cast<const uint4*>(k + src(1));
    pq1 = *reinterpret_cast<const uint4*>(q + src(1));
    pk2 = *reinterpret_cast<const uint4*>(k + src(2));
    pq2 = *reinterpret_cast<const uint4*>(q + src(2));
    pk3 = *reinterpret_cast<const uint4*>(k + src(3));
    pq3 = *reinterpret_cast<const uint4*>(q + src(3));
    if (wave == 0) {
      const size_t gi = size_t(x.t0 + min(lane, x.L - 1)) * HV + x.hv;
      pa = a[gi];
      pb = b[gi];
      pdt = dt_bias[x.hv];
      pal = A_log[x.hv];
    }
  };
  int u = blockIdx.x;
  Unit cur;
  if (u >= n_units || !locate(u, cur)) return;
  fetch(cur);
  for (;;) {
  const int slot = cur.slot, hv = cur.hv;
  const int L = cur.L;
  const int hq = hv / heads_per_qk;
  char* rec = blob + (size_t(slot) * HV + hv) * kBlob;

  // Raw rows (loaded a unit ahead): 16 threads per row, one 16-byte piece
  // each, into swizzled slots.
  {
    auto put = [&](int j, const uint4& wk, const uint4& wq) {
      const int item = tid + kPrepThreads * j;
      const int row = item >> 4, pc = item & 15;
      *reinterpret_cast<uint4*>(&rk[raw_off(row, 8 * pc)]) = wk;
      *reinterpret_cast<uint4*>(&rq[raw_off(row, 8 * pc)]) = wq;
    };
    put(0, pk0, pq0);
    put(1, pk1, pq1);
    put(2, pk2, pq2);
    put(3, pk3, pq3);
  }
  const uint16_t ua = pa, ub = pb;
  const float udt = pdt, ual = pal;
  // the next unit's loads, in flight while this one is processed
  Unit nxt;
  const int un = u + int(gridDim.x);
  const bool has_next = un < n_units && locate(un, nxt);
  if (has_next) fetch(nxt);

  // Gates of the chunk's tokens (reference PRE:1706-1722 and the chunk-local
  // cumsum of PRE:1721): lane = token.
  if (wave == 0) {
    constexpr float kLog2e = 1.44269504088896341f, kLn2 = 0.69314718055994531f;
    const float xa = bf16_bits_to_f32(ua) + udt;
    const float xb = bf16_bits_to_f32(ub);
    const float a_log_exp = expf(ual);
    float ld = 0.f, bt = 0.f;
    if (lane < L) {
      // softplus(x) = max(x, 0) + ln(1 + e^-|x|); sigmoid(y) = 1 / (1 + e^-y)
      const float sp = fmaxf(xa, 0.f) + kLn2 * __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-fabsf(xa) * kLog2e));
      ld = -a_log_exp * sp;
      bt = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-xb * kLog2e));
    }
    ld = wave_inclusive_scan(ld);
    const float l2 = ld * kLog2e;
    const float gl2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l2), L - 1));
    const float eg = __builtin_amdgcn_exp2f(l2);
    const float vals[5] = {l2, bt, eg, scale * eg, __builtin_amdgcn_exp2f(gl2 - l2)};
#pragma unroll
    for (int f = 0; f < 5; ++f) {
      gd[f * C + lane] = vals[f];
      reinterpret_cast<float*>(rec + BL_G)[f * C + lane] = vals[f];
    }
  }
  __syncthreads();
  if constexpr (kL2) {
    // Row factors (sum x^2 + 1e-6)^(-1/2): two threads per row of K, then Q.
    const int r = tid >> 1, hf = tid & 1;
    const uint16_t* src = r < C ? rk : rq;
    const int row = r & (C - 1);
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const uint4 w = *reinterpret_cast<const uint4*>(&src[raw_off(row, 64 * hf + 8 * p)]);
      float f[8];
      unpack_bf16x2(w.x, f[0], f[1]); unpack_bf16x2(w.y, f[2], f[3]);
      unpack_bf16x2(w.z, f[4], f[5]); unpack_bf16x2(w.w, f[6], f[7]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
    }
    ss += __shfl_xor(ss, 1);
    if (hf == 0) {
      const float fac = l2norm_rsqrt(ss);
      nrm[r] = fac;
      reinterpret_cast<float*>(rec + BL_N)[r] = fac;
    }
    __syncthreads();
  }
  const float* nk = nrm;
  const float* nq = nrm + C;
  const bool neg_scale = scale < 0.f;
  // The fp16 K rows of the chunk, once per qk-head (by its first v-head), in
  // the chain's LDS layout: [t][p32(k)], rows past the chunk end 0, scaled by
  // the row factor with the L2-norm option.
  if (hv % (HV / HQ) == 0) {
    char* kimg = blob + size_t(n_slots) * HV * kBlob + (size_t(slot) * HQ + hq) * kKcBytes;
#pragma unroll
    for (int j = 0; j < (C * D / 8) / kPrepThreads; ++j) {
      const int item = tid + kPrepThreads * j;
      const int row = item >> 4, cc = (item & 15) * 8;
      uint4 w = *reinterpret_cast<const uint4*>(&rk[raw_off(row, cc)]);
      if (row >= L) w = uint4{0u, 0u, 0u, 0u};
      float f[8];
      unpack_bf16x2(w.x, f[0], f[1]); unpack_bf16x2(w.y, f[2], f[3]);
      unpack_bf16x2(w.z, f[4], f[5]); unpack_bf16x2(w.w, f[6], f[7]);
      if constexpr (kL2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] *= nk[row];
      }
      _Float16* d = reinterpret_cast<_Float16*>(kimg) + row * KCLD + p32(cc);
      *reinterpret_cast<f16x4_t*>(d) = f16x4_t{(_Float16)f[0], (_Float16)f[1], (_Float16)f[2], (_Float16)f[3]};
      *reinterpret_cast<f16x4_t*>(d + 8) = f16x4_t{(_Float16)f[4], (_Float16)f[5], (_Float16)f[6], (_Float16)f[7]};
    }
  }
  const float scale_l2 = __log2f(fabsf(scale));

  // Per-lane swizzled offsets of the 8-column pieces read from a raw row r
  // with r % 16 == c: piece 4 ks + g sits in slot (4 ks + g) ^ c.
  int raw_lane[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) raw_lane[ks] = c * D + 8 * ((4 * ks + g) ^ c);

  // A tile = tril_strict(beta_i e^{gam_i - gam_j} K K^T), formed transposed
  // (K_j K_i^T) so that lane (g, c) holds row 16 ti + c, columns 16 tj + 4 g
  // .. +3.  Tiles of the diagonal 32-row blocks stay fp32 (the inverse's
  // input); the lower-left block is stored negated in fp16 (a chain operand).
  auto tile_A = [&](auto tile_c) {
    constexpr int ti = Tile16<decltype(tile_c)::value>::ti;
    constexpr int tj = Tile16<decltype(tile_c)::value>::tj;
    bf16x8_t fa[4], fb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      fa[ks] = ld16_bf(&rk[raw_lane[ks] + 16 * ti * D]);
      fb[ks] = ld16_bf(&rk[raw_lane[ks] + 16 * tj * D]);
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = mfma16_bf(fb[ks], fa[ks], acc);
    const float gr = gd[G_L2 + 16 * ti + c];
    float br = gd[G_BETA + 16 * ti + c];
    const f32x4 gcol = *reinterpret_cast<const f32x4*>(&gd[G_L2 + 16 * tj + 4 * g]);
    if constexpr (kL2) {
      br *= nk[16 * ti + c];
      acc *= *reinterpret_cast<const f32x4*>(&nk[16 * tj + 4 * g]);
    }
    f32x4 val;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      val[i] = br * __builtin_amdgcn_exp2f(gr - gcol[i]) * acc[i];
      if (ti == tj) val[i] = (c > 4 * g + i) ? val[i] : 0.f;
    }
    if (ti >= 2 && tj <= 1) {
      *reinterpret_cast<f16x4_t*>(&sAba[(16 * (ti - 2) + c) * BLD + 8 * g + 4 * tj]) =
          f16x4_t{(_Float16)-val[0], (_Float16)-val[1], (_Float16)-val[2], (_Float16)-val[3]};
    } else {
      *reinterpret_cast<f32x4*>(&sA[(16 * ti + c) * ALD + 16 * tj + 4 * g]) = val;
    }
  };
  // P tiles = scale tril_incl(e^{gam_i - gam_j} Q K^T), formed transposed like
  // the A tiles; |scale| enters the exponent, its sign the product.  The
  // tiles (ti, 2 s) and (ti, 2 s + 1) are formed together and their 8 p32
  // positions 32 s + 8 g .. +7 of row 16 ti + c go out as one 16-byte write
  // per lane (two 8-byte writes down 16 rows meet in the LDS banks); a tile
  // above the diagonal is written as zeros.
  auto tile_P_pair = [&](auto ti_c, auto s_c) {
    constexpr int ti = decltype(ti_c)::value;
    constexpr int tj0 = 2 * decltype(s_c)::value, tj1 = tj0 + 1;
    constexpr bool two = tj1 <= ti;
    bf16x8_t fa[4], fb0[4], fb1[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      fa[ks] = ld16_bf(&rq[raw_lane[ks] + 16 * ti * D]);
      fb0[ks] = ld16_bf(&rk[raw_lane[ks] + 16 * tj0 * D]);
      if constexpr (two) fb1[ks] = ld16_bf(&rk[raw_lane[ks] + 16 * tj1 * D]);
    }
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      acc0 = mfma16_bf(fb0[ks], fa[ks], acc0);
      if constexpr (two) acc1 = mfma16_bf(fb1[ks], fa[ks], acc1);
    }
    if (neg_scale) {
      acc0 = -acc0;
      acc1 = -acc1;
    }
    const float gr = gd[G_L2 + 16 * ti + c] + scale_l2;
    const f32x4 gcol0 = *reinterpret_cast<const f32x4*>(&gd[G_L2 + 16 * tj0 + 4 * g]);
    f32x4 gcol1 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (two) gcol1 = *reinterpret_cast<const f32x4*>(&gd[G_L2 + 16 * tj1 + 4 * g]);
    if constexpr (kL2) {
      acc0 *= nq[16 * ti + c] * *reinterpret_cast<const f32x4*>(&nk[16 * tj0 + 4 * g]);
      if constexpr (two) acc1 *= nq[16 * ti + c] * *reinterpret_cast<const f32x4*>(&nk[16 * tj1 + 4 * g]);
    }
    f16x8 val;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x0 = __builtin_amdgcn_exp2f(gr - gcol0[i]) * acc0[i];
      if (ti == tj0) x0 = (c >= 4 * g + i) ? x0 : 0.f;
      val[i] = (_Float16)x0;
      float x1 = 0.f;
      if constexpr (two) {
        x1 = __builtin_amdgcn_exp2f(gr - gcol1[i]) * acc1[i];
        if (ti == tj1) x1 = (c >= 4 * g + i) ? x1 : 0.f;
      }
      val[4 + i] = (_Float16)x1;
    }
    *reinterpret_cast<f16x8*>(&sP[(16 * ti + c) * TLD + 16 * tj0 + 8 * g]) = val;
  };
  switch (wave) {   // P tile pairs: (1, 0) (1, 1); (2, 0) (2, 1); (3, 0) (3, 1) and (0, 0); (3, 2) (3, 3) and (2, 2)
    case 0: tile_A(IC<0>{}); tile_A(IC<4>{}); tile_A(IC<8>{}); tile_P_pair(IC<1>{}, IC<0>{}); break;
    case 1: tile_A(IC<1>{}); tile_A(IC<5>{}); tile_A(IC<9>{}); tile_P_pair(IC<2>{}, IC<0>{}); break;
    case 2: tile_A(IC<2>{}); tile_A(IC<6>{}); tile_P_pair(IC<3>{}, IC<0>{}); tile_P_pair(IC<0>{}, IC<0>{}); break;
    default: tile_A(IC<3>{}); tile_A(IC<7>{}); tile_P_pair(IC<3>{}, IC<1>{}); tile_P_pair(IC<2>{}, IC<1>{}); break;
  }
  __syncthreads();

  auto put_frag = [&](int off, f16x8 x) {
    *reinterpret_cast<f16x8*>(rec + off + 16 * lane) = x;
  };
  if (wave == 0) {
    // Rows of the diagonal 16x16 blocks of Tm: lane group g inverts block g
    // by forward substitution in fp32 (lane = column), Tm[i] = e_i - sum_{j<i}
    // A[i][j] Tm[j] (the reference's diagonal-block solve, PRE:661-699).
    const float* Ab = &sA[(16 * g) * ALD + 16 * g];
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s0 = (i == c) ? 1.f : 0.f, s1 = 0.f;   // two partial sums halve the dependent chain
#pragma unroll
      for (int j4 = 0; j4 < i; j4 += 4) {
        const f32x4 arow = *reinterpret_cast<const f32x4*>(&Ab[i * ALD + j4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (j4 + e < i) {
            if ((j4 >> 2) & 1) s1 = fmaf(-arow[e], x[j4 + e], s1);
            else s0 = fmaf(-arow[e], x[j4 + e], s0);
          }
        }
      }
      x[i] = s0 + s1;
    }
    const int pc = p32(16 * g + c);
#pragma unroll
    for (int i = 0; i < 16; ++i) sTm[(16 * g + i) * TLD + pc] = (_Float16)x[i];
  } else {
    // P and -A_ba fragments, as the chain reads them: lane (g, c) gets row
    // 16 tb + c, p32 positions 32 p + 8 g .. + 7.
    constexpr int kPt[6] = {0, 1, 2, 2, 3, 3}, kPp[6] = {0, 0, 0, 1, 0, 1};
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      if (f % 3 != wave - 1) continue;
      if (f < 6) put_frag(BL_P + f * kFrag, ld16(&sP[(16 * kPt[f] + c) * TLD + 8 * g + 32 * kPp[f]]));
      else put_frag(BL_AB + (f - 6) * kFrag, ld16(&sAba[(16 * (f - 6) + c) * BLD + 8 * g]));
    }
  }
  __syncthreads();
  if (wave >= 2) {
    // 16-row merge inside the 32-row block at a0: T_{a0+16.., a0..} = -T_22 A_21 T_11.
    const int a0 = 32 * (wave - 2);
    const f32x4 a4 = *reinterpret_cast<const f32x4*>(&sA[(a0 + 16 + c) * ALD + a0 + 4 * g]);
    const f16x4_t fa = {(_Float16)a4[0], (_Float16)a4[1], (_Float16)a4[2], (_Float16)a4[3]};
    f16x4_t fb;
    const int pcb = p32(a0 + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) fb[e] = sTm[(a0 + 4 * g + e) * TLD + pcb];
    const f32x4 y = mfma16k16(fa, fb, f32x4{0.f, 0.f, 0.f, 0.f});
    const f16x4_t ft = *reinterpret_cast<const f16x4_t*>(&sTm[(a0 + 16 + c) * TLD + p32(a0 + 16 + 4 * g)]);
    const f16x4_t fy = {(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
    const f32x4 t21 = mfma16k16(ft, fy, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int i = 0; i < 4; ++i) sTm[(a0 + 16 + 4 * g + i) * TLD + pcb] = (_Float16)(-t21[i]);
  }
  __syncthreads();
  // Tm fragments: T_a rows 0-15 / 16-31 (p32 group 0), T_b rows 32-47 / 48-63 (group 1).
  {
    const int j = wave;
    const int off = j < 2 ? (16 * j + c) * TLD + 8 * g : (16 * j + c) * TLD + 32 + 8 * g;
    put_frag(BL_TM + j * kFrag, ld16(&sTm[off]));
  }
  __syncthreads();      // LDS of this unit read; the next unit overwrites it
  if (!has_next) break;
  u = un;
  cur = nxt;
  }
}

// ---------------------------------------------------------------------------
// State slice of one chain: R = 16 NRG state rows per workgroup.  Each group
// of 16 rows has a state wave and an output wave:
//   state wave  : X = beta (V - e^gam KS);  Vn_top = T_a X_top,
//                 Vn_bot = T_b (X_bot - A_ba Vn_top);  Vd = e^{gam_L - gam} Vn
//                 -> Vn to LDS;  S <- e^{gam_L} S + K^T Vd;  the new S as a bf16
//                 operand image to LDS;  KS = K S^T of the next chunk
//   output wave : O^T = scale e^gam S Q^T (S from the bf16 image), then (Vn
//                 from LDS) + Vn^T P^T, stored as bf16 rows
// and two copy waves stage, by HBM -> LDS copies issued NB - 1 chunks ahead
// into NB buffers each, the raw Q rows, the slice's V columns, the chunk's
// fp16 K image and its gate data.  The Tm, A_ba and P fragments of the chunk's
// workspace record go straight into the registers of the waves that use
// them, also two chunks ahead.  Two LDS barriers per chunk: after Vn is in
// LDS (by then the next chunk's copies have landed), and at the end of the
// chunk.  After the first, the state wave updates S and forms the next
// chunk's K S^T while the output wave finishes this chunk's rows, so the
// next chunk's X does not wait for the update.  State waves 0 .. NRG-1 and
// output waves NRG .. 2 NRG - 1 land on different SIMDs pairwise; the copy
// waves are 2 NRG and 2 NRG + 1.
template <int NRG>
struct SliceCfg {
  static constexpr int R = 16 * NRG;            // state rows per workgroup
  static constexpr int kThreads = 64 * (2 * NRG + 2);
  static constexpr int VS = R / 8;              // 16-byte slots per V row
  static constexpr int VRows = 1024 / (2 * R);  // V rows per 1 KB copy instruction
  // LDS buffer sets (copies are issued kNB - 1 chunks ahead)
  static constexpr int kNB = NRG == 1 ? 4 : 3;
  // chunks ahead that the record fragments are loaded (24 VGPRs a chunk),
  // and the register ring they rotate through (kNB is a multiple of it, so
  // the ring slot of a chunk follows from its LDS buffer set)
  static constexpr int kAhead = NRG == 1 ? 1 : kNB - 1;
  static constexpr int kFrRing = kAhead + 1;
  static_assert(kNB % kFrRing == 0, "ring slot from the buffer set");
};

// V slot swizzle of row t in a slice's LDS V rows (VS 16-byte slots per row):
// slot s holds piece s ^ vslot(t).  t mod VS, and at 32 rows (VS = 4) also
// 2 ((t / 4) mod 2): a transposing read cycle serves 8 rows with 4 lanes on
// 32 contiguous bytes (two slots) of each, and the rows t, t + 4 then take
// distinct slot pairs.
template <int VS>
__device__ __forceinline__ int vslot(int t) {
  return VS == 4 ? ((t & 3) ^ (((t >> 2) & 1) << 1)) : (t & (VS - 1));
}

//
// kH: the output waves also write the state entering every chunk, bf16, to
// hout[chunk_offset(n) + ch][hv][v][k] (slots at or past h_chunks skipped):
// the bf16 image of S they read for S Q^T is that state.
template <typename CuT, bool kL2, int NRG, bool kH>
__global__ __launch_bounds__(SliceCfg<NRG>::kThreads, 1) void gdn_prefill_slice_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ v, const float* __restrict__ h0,
    const CuT* __restrict__ cu_seqlens, int N, int T, int HQ, int HV,
    uint16_t* __restrict__ out, float* __restrict__ ht, char* __restrict__ ws, int nt_bound,
    uint16_t* __restrict__ hout, int h_chunks, int seam_room_) {
  using Cfg = SliceCfg<NRG>;
  constexpr int R = Cfg::R;
  constexpr int VS = Cfg::VS;
  constexpr int S = D / R;                      // slices per chain
  constexpr int NB = Cfg::kNB;
  __shared__ __align__(16) _Float16 Kc[NB][C * KCLD];
  __shared__ __align__(16) uint16_t rq[NB][C * D];
  __shared__ __align__(16) uint16_t rv[NB][C * R];
  __shared__ __align__(16) char gt[NB][kGateBytes];
  __shared__ __align__(16) f16x8 xch[NRG][2][64];   // Vn (2 fragments) per row group
  // bf16 operand image of each row group's state (the output waves' S Q^T),
  // written by the state wave after its update
  __shared__ __align__(16) bf16x8_t sSb[NRG][4][64];

  // Workgroup -> (unit = (sequence, qk-head), member m, slice s).  The G * S
  // workgroups of one unit read the same K, Q and (per member) records; they
  // get ids 8 apart, which puts them on one XCD (ids go round-robin over the
  // 8 XCDs), so only the first read of each line goes to HBM.  Units are
  // taken longest sequence first (order[], from the preparation launch):
  // unit position j of XCD x is sorted unit 8 j + x for even j and 8 j + 7 - x
  // for odd j, which evens out the work per XCD, and the workgroups that wait
  // for a CU land where the shortest of the first units ran.
  //
  // Workgroups past the chains' grid (ids from base_ids on) run the tails of
  // the seams in groups of G S workgroups, ids 8 apart on one XCD: group 2 u
  // of seam unit u = (seam j, qk-head hq) its zero-state tail chains, group
  // 2 u + 1 its transition chains.  Group gi sits on XCD (gi + off) mod 8,
  // off = seam_xcd_offset(n_units), and seam_room admits only seams whose
  // groups leave every XCD at most one workgroup per CU.
  const int G = HV / HQ;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const int* order = reinterpret_cast<const int*>(ws + order_offset(nt_bound, HQ, HV));
  const int n_units = N * HQ;
  const int base_ids = 8 * G * S * ((n_units + 7) / 8);
  // 0: the whole chain; 1: a seam's head; 2: its tail from a zero state; 3: its transition chain
  int role = 0, rank, m, s, hq;
  const int n_seams = seam_count(cu_seqlens, order, N, T, seam_room_);
  if (int(blockIdx.x) < base_ids) {
    const int xcd = blockIdx.x & 7, id_row = blockIdx.x >> 3;
    const int jx = id_row / (G * S);
    const int su = 8 * jx + ((jx & 1) ? 7 - xcd : xcd);
    if (su >= n_units) return;
    const int within = id_row - jx * (G * S);
    m = within / S;
    s = within - m * S;
    rank = su / HQ;
    hq = su - rank * HQ;
    if (rank < n_seams) role = 1;
  } else {
    const int e = int(blockIdx.x) - base_ids;
    const int xcd = e & 7, w = e >> 3;
    const int row = w / (G * S);
    const int gi = 8 * row + ((xcd - seam_xcd_offset(n_units)) & 7);
    if (gi >= 2 * n_seams * HQ) return;
    const int within = w - row * (G * S);
    role = 2 + (gi & 1);
    m = within / S;
    s = within - m * S;
    const int ux = gi >> 1;
    rank = ux / HQ;
    hq = ux - rank * HQ;
  }
  const int n = order[rank];
  const int hv = hq * G + m;
  const int vb = R * s;                         // first state row of the slice
  char* seam_ws = ws + seam_plan_offset(nt_bound, N, HQ, HV);   // the seam region
  int* plan = reinterpret_cast<int*>(seam_ws);
  if (blockIdx.x == 0 && tid == 0)
    for (int jj = n_seams; jj < seam_room_; ++jj) plan[kSeamPlanStride * jj + SP_SEQ] = -1;

  int bos, len;
  seq_bounds(cu_seqlens, n, T, bos, len);
  const size_t qk_stride = size_t(HQ) * D;
  const size_t v_stride = size_t(HV) * D;
  auto chunk_len = [&](int ch) { return min(C, len - ch * C); };
  const int coff = chunk_offset(cu_seqlens, n, T, lane);
  // The workspace holds nt_bound chunk slots, enough for every chunk of
  // well-formed cu_seqlens.  Ranges that overlap can count more chunks: the
  // chain then stops at the last slot the workspace holds (results
  // unspecified, every record and K image read in bounds).
  const int n_all = min((len + C - 1) / C, max(0, nt_bound - coff));
  // Chunks [ch0, ch0 + n_chunks) of the sequence: all of them, or a seam's
  // head [0, sp) or tail [sp, n_all).
  const int sp = seam_split_chunk(n_all);
  const int ch0 = role >= 2 ? sp : 0;
  const int n_chunks = role == 0 ? n_all : (role == 1 ? sp : n_all - sp);
  // workspace record of chunk ch of this chain
  auto record = [&](int ch) { return ws + (size_t(coff + ch) * HV + hv) * kBlob; };
  // seam state j of kind (0 head final, 1 tail final, 2 transition X^T) of this v-head
  auto seam_state = [&](int kind) {
    return reinterpret_cast<float*>(seam_ws + seam_state_offset(HV, rank, hv, kind));
  };
  // first OX row of seam `rank`: the tail tokens of the seams before it
  auto seam_ox_row = [&]() { return seam_rows_before(cu_seqlens, order, T, rank); };
  if (role == 1 && hq == 0 && m == 0 && s == 0 && tid == 0) {
    int* e = plan + kSeamPlanStride * rank;
    e[SP_SEQ] = n;
    e[SP_BOS] = bos;
    e[SP_LEN] = len;
    e[SP_SPLIT] = sp;
    e[SP_CHUNKS] = n_all;
    e[SP_OX_ROW] = seam_ox_row();
  }

  if (wave < 2 * NRG) {
    // ======================= state / output waves
    const bool out_role = wave >= NRG;
    const int r = out_role ? wave - NRG : wave;     // row group
    const int v0 = vb + 16 * r;                 // rows v0 + c
    const int vl = 16 * r;                      // the same, relative to the slice
    // kH: byte offset of this lane's 16 bytes in an h slot of the chain
    const uint32_t h_lane = uint32_t((v0 + c) * D + ((g & 1) ? 4 * (g + 3) : 4 * g)) * 2u;
    // Sacc[kb][i] = S[v0 + c][16 kb + 4 g + i]: the S^T accumulator tiles.
    // A seam's tail starts from zeros, its transition chain from the identity.
    f32x4 Sacc[8];
    const float* h0row = (h0 == nullptr || role >= 2) ? nullptr
                         : h0 + (size_t(n) * HV + hv) * size_t(D) * D + size_t(v0 + c) * D;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
      Sacc[kb] = (h0row && !out_role) ? *reinterpret_cast<const f32x4*>(h0row + 16 * kb + 4 * g)
                                      : f32x4{0.f, 0.f, 0.f, 0.f};
    if (role == 3) {
#pragma unroll
      for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) Sacc[kb][i] = (v0 + c == 16 * kb + 4 * g + i) ? 1.f : 0.f;
    }
    // the transition chain reads its v as zeros
    const int vmask = role == 3 ? 0 : -1;
    // Fragments of the chunk's record this wave multiplies with (state: T_a,
    // T_b, -A_ba; output: P), loaded kAhead chunks ahead.
    constexpr int kAhead = Cfg::kAhead;
    const int frag_base = out_role ? BL_P : BL_TM;
    constexpr int FR = Cfg::kFrRing;
    f16x8 fr[FR][6];
    auto load_frags = [&](int ch, f16x8 (&dst)[6]) {
      const char* rec = record(ch) + frag_base + 16 * lane;
#pragma unroll
      for (int f = 0; f < 6; ++f) dst[f] = *reinterpret_cast<const f16x8*>(rec + f * kFrag);
    };
    // (the chunk index is clamped: every chunk issues the same loads)
    const int last_ch = ch0 + n_chunks - 1;
    if (n_chunks > 0) {
#pragma unroll
      for (int a = 0; a < kAhead; ++a) load_frags(min(ch0 + a, last_ch), fr[a]);
    }
    // Per-lane element offsets of the two 4-column pieces of a Q fragment
    // (raw row 16 tb + c, columns 32 p + 4 g .. and 32 p + 16 + 4 g ..).
    const int sw = (g >> 1) ^ c;
    const int q_lane = c * D + 4 * (g & 1);

    // State update with the chunk's K^T fragments (transposing reads, a
    // k-block ahead) and Vd (state waves).
    auto update = [&](const _Float16* kc, float egL, const f16x8 (&vd)[2]) {
      auto load_kt = [&](int kb, f16x8 (&dst)[2]) {
        const int kq = p32(16 * kb + 4 * (c & 3));
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int tr0 = 32 * p + 4 * g + (c >> 2);
          const f16x4_t lo = ld_tr16(&kc[tr0 * KCLD + kq]);
          const f16x4_t hi = ld_tr16(&kc[(tr0 + 16) * KCLD + kq]);
          dst[p] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      };
      f16x8 fa[3][2];
      load_kt(0, fa[0]);
      load_kt(1, fa[1]);
#pragma unroll
      for (int kb = 0; kb < 8; ++kb) {
        if (kb + 2 < 8) load_kt(kb + 2, fa[(kb + 2) % 3]);
#pragma unroll
        for (int p = 0; p < 2; ++p) asm volatile("" : "+v"(fa[kb % 3][p]));
        Sacc[kb] *= egL;
#pragma unroll
        for (int p = 0; p < 2; ++p) Sacc[kb] = mfma16(fa[kb % 3][p], vd[p], Sacc[kb]);
      }
    };

    // K S^T with the rows of S this wave holds (fp16 operands: the fp16 K
    // image, S packed from the accumulators), K fragments a column block ahead.
    f32x4 KS[4];
    auto ks_of = [&](const _Float16* kcb, f32x4 (&ks_out)[4]) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) ks_out[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
      f16x8 kf[3][4];                         // K rows 16 tb + c, p32 positions 32 p + 8 g ..
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) kf[p][tb] = ld16(&kcb[(16 * tb + c) * KCLD + 32 * p + 8 * g]);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        if (p + 2 < 4) {
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) kf[(p + 2) % 3][tb] = ld16(&kcb[(16 * tb + c) * KCLD + 32 * (p + 2) + 8 * g]);
        }
        const f16x8 sb = pack2(Sacc[2 * p], Sacc[2 * p + 1]);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          asm volatile("" : "+v"(kf[p % 3][tb]));
          ks_out[tb] = mfma16(kf[p % 3][tb], sb, ks_out[tb]);
        }
      }
    };
    // One chunk; b3c (0, 1, 2) is the buffer set as a compile-time constant,
    // so every LDS address is a loop-invariant lane offset plus an immediate.
    auto chunk = [&](auto b3c, auto rolec, int jj) __attribute__((always_inline)) {
      constexpr int b3 = decltype(b3c)::value;
      constexpr bool kOut = decltype(rolec)::value != 0;
      const int ch = ch0 + jj;                  // the chunk; jj its place in this chain's run
      const int L = chunk_len(ch);
      const float* gd = reinterpret_cast<const float*>(gt[b3]);
      const _Float16* kc = Kc[b3];
      const float egL = gd[G_EG + L - 1];
      load_frags(min(ch + kAhead, last_ch), fr[(b3 + kAhead) % FR]);
      if constexpr (!kOut) {
        // K S^T of this chunk was formed at the end of the chunk before
        // ---- X = beta (V - e^gam K S^T).  V[16 tb + 4 g + i][v0 + c] by one
        //      transposing read per tb: lane 4 mm + j reads columns vl + 4 j
        //      .. +3 of row 16 tb + 4 g + mm.
        {
          const int mm = c >> 2, j = c & 3;
          const int col = vl + 4 * j;
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const int t = 16 * tb + 4 * g + mm;
            const i16x4_t vv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4_t*)&rv[b3][t * R + 8 * ((col >> 3) ^ vslot<VS>(t)) + (col & 7)]) &
                i16x4_t{short(vmask), short(vmask), short(vmask), short(vmask)};
            const f32x4 eg = *reinterpret_cast<const f32x4*>(&gd[G_EG + 16 * tb + 4 * g]);
            const f32x4 bt = *reinterpret_cast<const f32x4*>(&gd[G_BETA + 16 * tb + 4 * g]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              KS[tb][i] = bt[i] * (bf16_bits_to_f32(uint16_t(vv[i])) - eg[i] * KS[tb][i]);
          }
        }
        // ---- Vn = Tm X in 32-row blocks: Vn_top = T_a X_top, Vn_bot = T_b (X_bot - A_ba Vn_top)
        f16x8 vd[2];
        {
          const f16x8* tf = fr[b3 % FR];        // T_a rows 0-15, 16-31; T_b rows 32-47, 48-63; -A_ba
          f32x4 ed[4];
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) ed[tb] = *reinterpret_cast<const f32x4*>(&gd[G_ED + 16 * tb + 4 * g]);
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          f32x4 Vn[4];
          f16x8 xb = pack2(KS[0], KS[1]);
          Vn[0] = mfma16(tf[0], xb, z);
          Vn[1] = mfma16(tf[1], xb, z);
          const f16x8 vn0 = pack2(Vn[0], Vn[1]);
          KS[2] = mfma16(tf[4], vn0, KS[2]);
          KS[3] = mfma16(tf[5], vn0, KS[3]);
          vd[0] = pack2(Vn[0] * ed[0], Vn[1] * ed[1]);
          xb = pack2(KS[2], KS[3]);
          Vn[2] = mfma16(tf[2], xb, z);
          Vn[3] = mfma16(tf[3], xb, z);
          const f16x8 vn1 = pack2(Vn[2], Vn[3]);
          vd[1] = pack2(Vn[2] * ed[2], Vn[3] * ed[3]);
          xch[r][0][lane] = vn0;
          xch[r][1][lane] = vn1;
        }
        lds_barrier();                          // Vn of every row group in LDS
        update(kc, egL, vd);
        // the new state's bf16 image for the output wave, and K S^T of the next chunk
#pragma unroll
        for (int p = 0; p < 4; ++p) sSb[r][p][lane] = pack2_bf(Sacc[2 * p], Sacc[2 * p + 1]);
        if (jj + 1 < n_chunks) ks_of(Kc[(b3 + 1) % NB], KS);
      } else {
        // ---- O^T = S Q^T (transposed output tile: lane (g, c) of OT[tb] holds
        //      token 16 tb + c, state rows v0 + 4 g .. +3)
        f32x4 OT[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) OT[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto load_q = [&](int p, bf16x8_t (&dst)[4]) {
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const uint16_t* qr = &rq[b3][q_lane + 16 * tb * D];
            const bf16x4_t lo = *reinterpret_cast<const bf16x4_t*>(&qr[8 * ((4 * p) ^ sw)]);
            const bf16x4_t hi = *reinterpret_cast<const bf16x4_t*>(&qr[8 * ((4 * p + 2) ^ sw)]);
            dst[tb] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          }
        };
        bf16x8_t qf[2][4];
        load_q(0, qf[0]);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          if (p + 1 < 4) load_q(p + 1, qf[(p + 1) & 1]);
          const bf16x8_t sbf = sSb[r][p][lane];
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            asm volatile("" : "+v"(qf[p & 1][tb]));
            OT[tb] = mfma16_bf(sbf, qf[p & 1][tb], OT[tb]);
          }
          if constexpr (kH) {
            // Lane (g, c) holds row v0 + c, 4-column pieces g and g + 4 of
            // column block p; v_permlane16_swap trades the odd 16-lane rows'
            // first piece for the even rows' second, which leaves 16
            // contiguous bytes per lane (pieces g, g + 1 for even g, g + 3,
            // g + 4 for odd g): one 16-byte store covers 16 rows x 64 bytes.
            // (Whole lines two blocks at a time, store_state_lines, are
            // slower here: the extra lane exchange sits on this wave's path,
            // and at few chains the half lines cost little in HBM.)
            if (coff + ch < h_chunks) {
              char* hb = reinterpret_cast<char*>(hout) + (size_t(coff + ch) * HV + hv) * size_t(D * D * 2);
              const u32x4_t w = __builtin_bit_cast(u32x4_t, sbf);
              const auto lo = __builtin_amdgcn_permlane16_swap(w[0], w[2], false, false);
              const auto hi = __builtin_amdgcn_permlane16_swap(w[1], w[3], false, false);
              store_b128_saddr(hb, h_lane + uint32_t(64 * p), u32x4_t{lo[0], hi[0], lo[1], hi[1]});
            }
          }
        }
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          float egs = gd[G_EGS + 16 * tb + c];
          if constexpr (kL2) egs *= gd[(BL_N - BL_G) / 4 + C + 16 * tb + c];
          OT[tb] *= egs;
        }
        lds_barrier();                          // Vn, Vd of every row group in LDS
        f16x8 vn[2];
        vn[0] = xch[r][0][lane];
        vn[1] = xch[r][1][lane];
        // ---- + Vn^T P^T, then the rows to HBM
        {
          const f16x8* pf = fr[b3 % FR];        // P (token block, column block) 00 10 20 21 30 31
          constexpr int kPt[6] = {0, 1, 2, 2, 3, 3}, kPp[6] = {0, 0, 0, 1, 0, 1};
#pragma unroll
          for (int f = 0; f < 6; ++f) OT[kPt[f]] = mfma16(vn[kPp[f]], pf[f], OT[kPt[f]]);
          // the chunk's L rows as one buffer: stores of rows past L are dropped
          // (a transition chain's rows go to its seam's OX rows, cut at their end)
          uint16_t* obase = out + size_t(bos + ch * C) * v_stride;
          uint32_t orow_n = uint32_t(L);
          if (role == 3) {
            const int r0 = seam_ox_row() + (ch - ch0) * C;
            obase = reinterpret_cast<uint16_t*>(seam_ws + seam_ox_offset(seam_slots(N), HV)) + size_t(r0) * v_stride;
            orow_n = uint32_t(max(0, min(L, seam_ox_rows(N, T) - r0)));
          }
          const __amdgpu_buffer_rsrc_t orows =
              uniform_buffer(obase, orow_n * uint32_t(v_stride) * 2u);
          const uint32_t ocol = uint32_t(hv * D + v0 + 4 * g) * 2u;
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const int t = 16 * tb + c;
            buffer_store_b64(orows, t < L ? uint32_t(t) * uint32_t(v_stride) * 2u + ocol : kBufferDrop,
                             cvt_pk_bf16(OT[tb][0], OT[tb][1]), cvt_pk_bf16(OT[tb][2], OT[tb][3]));
          }
        }
      }
      lds_barrier();                            // chunk ch+1 staged; buffers of ch free
    };
    // The chunk loop of one role.  Its body issues the same vector memory
    // instructions on every path (clamped record loads; output rows as
    // buffer stores), so the compiler's waits for the record fragments count
    // exactly the loads issued after them instead of draining the queue;
    // the last n_chunks % NB chunks run after the loop.
    auto run = [&](auto rolec) __attribute__((always_inline)) {
      constexpr bool kOut = decltype(rolec)::value != 0;
      if constexpr (!kOut) {
#pragma unroll
        for (int p = 0; p < 4; ++p) sSb[r][p][lane] = pack2_bf(Sacc[2 * p], Sacc[2 * p + 1]);
      }
      lds_barrier();                            // chunk 0 staged, the initial state's image written
      if constexpr (!kOut) ks_of(Kc[0], KS);
      int ch = 0;
      for (; ch + NB <= n_chunks; ch += NB) {
        chunk(IC<0>{}, rolec, ch);
        chunk(IC<1>{}, rolec, ch + 1);
        chunk(IC<2>{}, rolec, ch + 2);
        if constexpr (NB > 3) chunk(IC<(NB > 3 ? 3 : 0)>{}, rolec, ch + 3);
      }
      if (ch < n_chunks) chunk(IC<0>{}, rolec, ch);
      if (ch + 1 < n_chunks) chunk(IC<1>{}, rolec, ch + 1);
      if (NB > 3 && ch + 2 < n_chunks) chunk(IC<2>{}, rolec, ch + 2);
    };
    if (n_chunks > 0) {
      if (out_role) run(IC<1>{});
      else run(IC<0>{});
    }
    if (!out_role) {
      if (role == 3) {                          // X stored transposed: X^T[k][v]
        float* dst = seam_state(2);
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[size_t(16 * kb + 4 * g + i) * D + v0 + c] = Sacc[kb][i];
      } else {
        float* dst = (role == 0 ? ht + (size_t(n) * HV + hv) * size_t(D) * D : seam_state(role - 1)) +
                     size_t(v0 + c) * D;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) *reinterpret_cast<f32x4*>(dst + 16 * kb + 4 * g) = Sacc[kb];
      }
    }
  } else {
    // ======================= copy waves
    // Copy wave 0 stages the raw Q rows and the gate data, copy wave 1 the fp16
    // K image and the slice's V columns: about 20 copies a chunk each, so the
    // NB - 1 chunks in flight stay within what one wave's vmcnt counts (63).
    // Per-lane byte offsets from a full chunk's first row: raw Q rows (4 rows
    // per instruction, lane l -> row 4 j + l / 16, slot l % 16 holding piece
    // (l % 16) ^ row) and V columns (lane l -> row VRows j + l / VS, slot
    // l % VS holding piece (l % VS) ^ (row % VS)).
    const char* kc0 = ws + size_t(nt_bound) * HV * kBlob + (size_t(coff) * HQ + hq) * kKcBytes;
    const uint32_t lane16 = 16u * uint32_t(lane);
    // LDS byte address of a buffer, as a wave-uniform scalar.
    auto lds_u32 = [](const void* p) {
      return __builtin_amdgcn_readfirstlane(
          (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p);
    };
    auto run_copies = [&](auto cwc) __attribute__((always_inline)) {
      constexpr int CW = decltype(cwc)::value;
      constexpr int kCopiesW = CW == 0 ? 16 + kGateCopies : kKcCopies + VS;   // copy instructions per chunk
      static_assert(2 * kCopiesW <= 63 && (NB - 1) * kCopiesW <= 63, "copies in flight within vmcnt");
      uint32_t q_off[16], v_off[VS];
      if constexpr (CW == 0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int row = 4 * j + (lane >> 4);
          q_off[j] = uint32_t(row) * uint32_t(qk_stride * 2) + uint32_t((lane & 15) ^ (row & 15)) * 16u;
        }
      } else {
#pragma unroll
        for (int j = 0; j < VS; ++j) {
          const int row = Cfg::VRows * j + lane / VS;
          v_off[j] = uint32_t(row) * uint32_t(v_stride * 2) + uint32_t((lane % VS) ^ vslot<VS>(row)) * 16u;
        }
      }
      auto issue_copies = [&](int jj) {
        const int ch = ch0 + jj;                // the chunk; jj its place in the run
        const int t0 = bos + ch * C, L = chunk_len(ch);
        const int b3 = jj % NB;
        if constexpr (CW == 0) {
          const uint32_t lq = lds_u32(rq[b3]);
          if (L == C) {
            const char* qb = reinterpret_cast<const char*>(q + size_t(t0) * qk_stride + size_t(hq) * D);
#pragma unroll
            for (int j = 0; j < 16; ++j) dma16(qb, q_off[j], lq + uint32_t(kFrag * j));
          } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int row = 4 * j + (lane >> 4);
              const int src_piece = (lane & 15) ^ (row & 15);
              lds_dma16(q + size_t(t0 + min(row, L - 1)) * qk_stride + size_t(hq) * D + 8 * src_piece,
                        &rq[b3][4 * j * D]);
            }
          }
          const char* gsrc = record(ch) + BL_G;
          const uint32_t lg = lds_u32(gt[b3]);
#pragma unroll
          for (int j = 0; j < kGateCopies; ++j)
            if (j < kGateCopies - 1 || kFrag * j + 16 * lane < kGateBytes)
              dma16(gsrc + kFrag * j, lane16, lg + uint32_t(kFrag * j));
        } else {
          const uint32_t lv = lds_u32(rv[b3]);
          if (L == C) {
            const char* vbp = reinterpret_cast<const char*>(v + size_t(t0) * v_stride + size_t(hv) * D + vb);
#pragma unroll
            for (int j = 0; j < VS; ++j) dma16(vbp, v_off[j], lv + uint32_t(kFrag * j));
          } else {
#pragma unroll
            for (int j = 0; j < VS; ++j) {
              const int row = Cfg::VRows * j + lane / VS;
              const int src_piece = (lane % VS) ^ vslot<VS>(row);
              lds_dma16(v + size_t(t0 + min(row, L - 1)) * v_stride + size_t(hv) * D + vb + 8 * src_piece,
                        &rv[b3][Cfg::VRows * j * R]);
            }
          }
          const char* kcs = kc0 + size_t(ch) * HQ * kKcBytes;
          const uint32_t lk = lds_u32(Kc[b3]);
#pragma unroll
          for (int j = 0; j < kKcCopies; ++j) dma16(kcs + kFrag * j, lane16, lk + uint32_t(kFrag * j));
        }
      };
      // copies(ch) land before the barrier that ends chunk ch - 1: at most
      // (NB - 2) later chunks' copies are still in flight then.
      auto wait_ahead = [&](int later) {        // wait until `later` chunks' copies remain
        if (later >= 2 && NB > 3) wait_vm<2 * kCopiesW>();
        else if (later >= 1) wait_vm<kCopiesW>();
        else wait_vm<0>();
      };
      if (n_chunks > 0) {
#pragma unroll
        for (int a = 0; a < NB - 1; ++a)
          if (a < n_chunks) issue_copies(a);
        wait_ahead(min(n_chunks, NB - 1) - 1);  // copies(0) landed
        lds_barrier();
      }
      for (int ch = 0; ch < n_chunks; ++ch) {
        // the chain reads chunk ch; copies(ch+1 .. ch+NB-2) are in flight,
        // copies(ch+NB-1) go into the buffers chunk ch-1 used
        if (ch + NB - 1 < n_chunks) issue_copies(ch + NB - 1);
        // copies(ch+1) land before the middle barrier: the state waves form
        // K S^T of chunk ch+1 after it
        wait_ahead(min(n_chunks - 1, ch + NB - 1) - (ch + 1));
        lds_barrier();                          // Vn exchange of chunk ch
        lds_barrier();
      }
    };
    if (wave == 2 * NRG) run_copies(IC<0>{});
    else run_copies(IC<1>{});
  }
}

// ---------------------------------------------------------------------------
// Seam pass, after the chains.  For seam j and v-head hv: pieces
// 0 .. kSeamStatePieces - 1 write 16 rows each of the sequence's final state
// S_sp X + S0; piece p >= kSeamStatePieces adds OX_c S_sp^T to the
// outputs of kSeamGroupChunks tail chunks c from sp + kSeamGroupChunks
// (p - kSeamStatePieces) on (the part of the tail outputs that depends on the
// state the head reached).  The final state takes fp32-accurate products
// (each fp32 operand split into two fp16 parts, three 16x16x16 MFMA
// products); the outputs bf16 products, as the output path does.  Four waves.
// A state piece issues all its loads before its first MFMA.  A tail piece
// stages S_sp once, as bf16 MFMA A fragments in LDS; wave w then owns tokens
// 16 w .. 16 w + 15 of each chunk across all 128 rows v (its OX rows read
// once), passes its corrections through LDS so that the outputs are read
// and written as whole rows, and loads the next chunk's OX rows and outputs
// while it works on a chunk.
constexpr int kSeamThreads = 256;
constexpr int kSeamStatePieces = D / 16;
constexpr int kSeamGroupChunks = 2;

__device__ __forceinline__ void split_f16(const f32x4& x, f16x4_t& hi, f16x4_t& lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hi[i] = (_Float16)x[i];
    lo[i] = (_Float16)(x[i] - (float)hi[i]);
  }
}

__host__ __device__ inline int seam_pieces(int max_tail_chunks) {
  return kSeamStatePieces + (max_tail_chunks + kSeamGroupChunks - 1) / kSeamGroupChunks;
}

__global__ __launch_bounds__(kSeamThreads) void gdn_prefill_seam_kernel(
    const char* __restrict__ region, int HV, int k_slots, int ox_rows, int seams, int pieces,
    uint16_t* __restrict__ out, float* __restrict__ ht) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int g = lane >> 4, c = lane & 15;
  // Workgroup -> (seam j, v-head hv, piece): the pieces of one (j, hv) get ids
  // 8 apart, which puts them on one XCD (ids go round-robin over the 8 XCDs),
  // so its three states come from HBM into one L2 once.
  const int xcd = int(blockIdx.x) & 7, id_row = int(blockIdx.x) >> 3;
  const int jh = 8 * (id_row / pieces) + xcd;
  const int piece = id_row - (id_row / pieces) * pieces;
  const int j = jh / HV, hv = jh - j * HV;
  if (j >= seams || j >= k_slots) return;
  // the plan entry of seam slot j (sequence or -1, bounds, split, first OX
  // row), one load
  const int* plan = reinterpret_cast<const int*>(region);
  const int pe = plan[kSeamPlanStride * j + (lane & (kSeamPlanStride - 1))];   // lane f: field f
  const int n = __builtin_amdgcn_readlane(pe, SP_SEQ);
  if (n < 0) return;
  const int bos = __builtin_amdgcn_readlane(pe, SP_BOS), len = __builtin_amdgcn_readlane(pe, SP_LEN);
  const int sp = __builtin_amdgcn_readlane(pe, SP_SPLIT), n_all = __builtin_amdgcn_readlane(pe, SP_CHUNKS);
  const int ox_row0 = __builtin_amdgcn_readlane(pe, SP_OX_ROW);
  if (piece >= kSeamStatePieces + (n_all - sp + kSeamGroupChunks - 1) / kSeamGroupChunks) return;
  auto state = [&](int kind) {
    return reinterpret_cast<const float*>(region + seam_state_offset(HV, j, hv, kind));
  };
  const float* Ssp = state(0);
  if (piece < kSeamStatePieces) {
    // S_L[v][k] = sum_k' S_sp[v][k'] X[k'][k] + S0[v][k] for rows v of block
    // tm = piece; wave w: column blocks tn = 2 w, 2 w + 1
    const int tm = piece;
    const float* S0 = state(1);
    const float* XT = state(2);
    f32x4 sa[8], xb[2][8], acc[2];
#pragma unroll
    for (int tk = 0; tk < 8; ++tk) {
      sa[tk] = *reinterpret_cast<const f32x4*>(&Ssp[size_t(16 * tm + c) * D + 16 * tk + 4 * g]);
#pragma unroll
      for (int u = 0; u < 2; ++u)
        xb[u][tk] = *reinterpret_cast<const f32x4*>(&XT[size_t(16 * (2 * wave + u) + c) * D + 16 * tk + 4 * g]);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[u][i] = S0[size_t(16 * tm + 4 * g + i) * D + 16 * (2 * wave + u) + c];
#pragma unroll
    for (int tk = 0; tk < 8; ++tk) {
      f16x4_t ah, al;
      split_f16(sa[tk], ah, al);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        f16x4_t bh, bl;
        split_f16(xb[u][tk], bh, bl);
        acc[u] = mfma16k16(ah, bh, acc[u]);
        acc[u] = mfma16k16(ah, bl, acc[u]);
        acc[u] = mfma16k16(al, bh, acc[u]);
      }
    }
    float* dst = ht + (size_t(n) * HV + hv) * size_t(D) * D;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[size_t(16 * tm + 4 * g + i) * D + 16 * (2 * wave + u) + c] = acc[u][i];
    return;
  }
  // Tail chunks ch of this group: dO^T[v][t] = sum_k' S_sp[v][k'] OX[t][k'],
  // added to out[t][hv][v].  S_sp as bf16 A fragments in LDS: fragment
  // (tm, tk) (rows 16 tm .., k' 32 tk ..) at 1 KiB steps, lane (g, c) of it
  // (row 16 tm + c, k' 32 tk + 8 g .. + 7) at 16 g + c 16-byte slots.
  __shared__ __align__(16) bf16x8_t sA[8 * 4 * 64];
  const int tid = threadIdx.x;
  static_assert(8 * 4 * 64 % kSeamThreads == 0, "staging");
#pragma unroll 4
  for (int i = 0; i < 8 * 4 * 64 / kSeamThreads; ++i) {
    const int idx = tid + kSeamThreads * i;       // (tm, tk, g, c), c fastest: < 2048
    const int cc = idx & 15, gg = (idx >> 4) & 3, tk = (idx >> 6) & 3, tm = idx >> 8;
    const float* sr = &Ssp[size_t(16 * tm + cc) * D + 32 * tk + 8 * gg];
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(sr);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(sr + 4);
    sA[(tm * 4 + tk) * 64 + gg * 16 + cc] =
        bf16x8_t{(__bf16)s0[0], (__bf16)s0[1], (__bf16)s0[2], (__bf16)s0[3],
                 (__bf16)s1[0], (__bf16)s1[1], (__bf16)s1[2], (__bf16)s1[3]};
  }
  const int chb = sp + (piece - kSeamStatePieces) * kSeamGroupChunks;
  const int che = min(n_all, chb + kSeamGroupChunks);
  const size_t v_stride = size_t(HV) * D;
  const uint16_t* OX = reinterpret_cast<const uint16_t*>(region + seam_ox_offset(k_slots, HV));
  // Each wave's corrections of a chunk, fp32 [token 16][v 128] (rows padded
  // to 132 floats: the 16-byte writes of 16 rows hit distinct banks), so the
  // outputs are read and written as whole rows: lane l takes row 4 j + l / 16,
  // 8 values from 8 (l % 16), j = 0..3.
  constexpr int kDLD = D + 4;
  __shared__ __align__(16) float sD[4][16 * kDLD];
  float* dW = sD[wave];
  const int t = 16 * wave + c;                    // this lane's token of the chunk (B column)
  const int q8 = 8 * (lane & 15);                 // this lane's 8 columns in the row-major passes
  // the chunk's token tt exists: inside the sequence and the OX region
  auto valid = [&](int ch, int tt) {
    return tt < min(C, len - ch * C) && ox_row0 + (ch - sp) * C + tt < ox_rows;
  };
  auto out_row = [&](int ch, int j) {
    return reinterpret_cast<uint4*>(out + size_t(bos + ch * C + 16 * wave + 4 * j + (lane >> 4)) * v_stride +
                                    size_t(hv) * D + q8);
  };
  uint4 ob[2][4], ov[2][4];
  auto load = [&](int ch, uint4 (&obb)[4], uint4 (&ovb)[4]) {
    const int orow = min(ox_row0 + (ch - sp) * C + t, ox_rows - 1);   // rows past the region are never used
#pragma unroll
    for (int tk = 0; tk < 4; ++tk)
      obb[tk] = *reinterpret_cast<const uint4*>(&OX[size_t(orow) * v_stride + size_t(hv) * D + 32 * tk + 8 * g]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      ovb[j] = valid(ch, 16 * wave + 4 * j + (lane >> 4)) ? *out_row(ch, j) : uint4{0u, 0u, 0u, 0u};
  };
  if (chb < che) load(chb, ob[0], ov[0]);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSeamGroupChunks; ++i) {
    const int ch = chb + i;
    if (ch >= che) break;
    if (ch + 1 < che) load(ch + 1, ob[(i + 1) & 1], ov[(i + 1) & 1]);
#pragma unroll
    for (int tm = 0; tm < 8; ++tm) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tk = 0; tk < 4; ++tk)
        acc = mfma16_bf(sA[(tm * 4 + tk) * 64 + lane], __builtin_bit_cast(bf16x8_t, ob[i & 1][tk]), acc);
      // acc[e]: v = 16 tm + 4 g + e, token c of this wave's 16
      *reinterpret_cast<f32x4*>(&dW[c * kDLD + 16 * tm + 4 * g]) = acc;
    }
    // the wave reads back what its lanes wrote (LDS keeps one wave's order)
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 4 * j + (lane >> 4);
      if (valid(ch, 16 * wave + r)) {
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(&dW[r * kDLD + q8]);
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(&dW[r * kDLD + q8 + 4]);
        const uint4 o = ov[i & 1][j];
        float f[8];
        unpack_bf16x2(o.x, f[0], f[1]);
        unpack_bf16x2(o.y, f[2], f[3]);
        unpack_bf16x2(o.z, f[4], f[5]);
        unpack_bf16x2(o.w, f[6], f[7]);
        *out_row(ch, j) = uint4{cvt_pk_bf16(f[0] + d0[0], f[1] + d0[1]), cvt_pk_bf16(f[2] + d0[2], f[3] + d0[3]),
                                cvt_pk_bf16(f[4] + d1[0], f[5] + d1[1]), cvt_pk_bf16(f[6] + d1[2], f[7] + d1[3])};
      }
    }
    asm volatile("" ::: "memory");
  }
}

}  // namespace

namespace gdn {

int prefill_split_seam_room(int N, int HQ, int HV, int slices, int cus) {
  return seam_room(N, HQ, HV, slices, cus);
}

int prefill_split_seam_span(const int* chunks_desc, int N, int room, int* seams) {
  int span = 0;
  const int k = seam_choice([&](int r) { return chunks_desc[r]; }, N, room, &span);
  if (seams) *seams = k;
  return span;
}

int prefill_seam_pass(char* region, int HV, int k_slots, int ox_rows, int seams, int max_tail_chunks,
                      uint16_t* out, float* final_state, hipStream_t st) {
  if (seams <= 0) return GDN_OK;
  const unsigned pieces = unsigned(seam_pieces(max_tail_chunks));
  const unsigned pairs = unsigned(seams) * unsigned(HV);
  const dim3 grid{8u * pieces * ((pairs + 7u) / 8u), 1u, 1u};
  hipLaunchKernelGGL(gdn_prefill_seam_kernel, grid, dim3(kSeamThreads), 0, st, region, HV, k_slots, ox_rows,
                     seams, int(pieces), out, final_state);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GDN_OK : -int(e);
}

}  // namespace gdn

namespace {

int device_cu_count();

template <typename CuT, bool kL2, int NRG>
void launch_slices(dim3 grid, hipStream_t st, const uint16_t* q, const uint16_t* v, const float* state,
                   const CuT* cu, int N, int T, int HQ, int HV, uint16_t* out, float* final_state,
                   char* ws, int nt_bound, uint16_t* h, int h_chunks, int room) {
  if (h != nullptr)
    hipLaunchKernelGGL((gdn_prefill_slice_kernel<CuT, kL2, NRG, true>), grid, dim3(SliceCfg<NRG>::kThreads), 0,
                       st, q, v, state, cu, N, T, HQ, HV, out, final_state, ws, nt_bound, h, h_chunks, 0);
  else
    hipLaunchKernelGGL((gdn_prefill_slice_kernel<CuT, kL2, NRG, false>), grid, dim3(SliceCfg<NRG>::kThreads), 0,
                       st, q, v, state, cu, N, T, HQ, HV, out, final_state, ws, nt_bound, nullptr, 0, room);
}

template <typename CuT, bool kL2>
int launch_split_t(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* state,
                   const float* A_log, const uint16_t* a, const float* dt_bias, const uint16_t* b,
                   const CuT* cu, int N, int T, int HQ, int HV, float scale, uint16_t* out,
                   float* final_state, int slices, char* ws, uint16_t* h, int h_chunks, bool no_seams,
                   hipStream_t st) {
  const int nt_bound = T / C + N;
  if (nt_bound > 0) {
    // persistent workgroups, two per CU (75.5 KB of LDS each)
    const long long units = (long long)nt_bound * HV;
    const int cus = device_cu_count();
    const long long wgs = std::min<long long>(units, 2LL * (cus > 0 ? cus : 256));
    hipLaunchKernelGGL((gdn_prefill_prep_kernel<CuT, kL2>), dim3(unsigned(wgs)), dim3(kPrepThreads), 0,
                       st, q, k, A_log, a, dt_bias, b, cu, N, T, HQ, HV, scale, ws, nt_bound);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return -int(e);
  }
  const unsigned units = unsigned(N) * unsigned(HQ);
  const unsigned G = unsigned(HV / HQ);
  // Seams (time splits of the longest chains) use the CUs the slices leave
  // idle; not with the per-chunk states (h), which the tails cannot give.
  const int cus = device_cu_count();
  const int room = (h == nullptr && !no_seams) ? seam_room(N, HQ, HV, slices, cus > 0 ? cus : 256) : 0;
  const unsigned base = 8u * G * unsigned(slices) * ((units + 7u) / 8u);
  const unsigned seam_groups = 2u * unsigned(room) * unsigned(HQ);
  const unsigned extra = 8u * G * unsigned(slices) * ((seam_groups + 7u) / 8u);
  const dim3 grid{base + extra, 1u, 1u};
  switch (slices) {
    case 8:
      launch_slices<CuT, kL2, 1>(grid, st, q, v, state, cu, N, T, HQ, HV, out, final_state, ws, nt_bound,
                                 h, h_chunks, room);
      break;
    case 4:
      launch_slices<CuT, kL2, 2>(grid, st, q, v, state, cu, N, T, HQ, HV, out, final_state, ws, nt_bound,
                                 h, h_chunks, room);
      break;
    default:
      return GDN_ERR_SHAPE;
  }
  if (room > 0) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return -int(e);
    // pieces: the final state's blocks, then the longest possible tail
    const int r = prefill_seam_pass(ws + seam_plan_offset(nt_bound, N, HQ, HV), HV, seam_slots(N),
                                    seam_ox_rows(N, T), room, (nt_bound + 1) / 2 + 1, out, final_state, st);
    if (r != GDN_OK) return r;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GDN_OK : -int(e);
}

// Workspace of the allocation-free split entry point: a device array of
// kScratchBytes that every GPU the library runs on holds until the process
// ends.  Host code uses it only through the per-device address that
// hipGetSymbolAddress returns (the array's name is a host-side stand-in).
// Calls on one GPU share it: calls that overlap on one GPU race.  Nothing in
// it has to start at zero (the preparation launch writes every byte the
// slice launch reads).
constexpr size_t kScratchBytes = size_t(32) << 20;
__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Address of `scratch` on the current device (looked up once per device), or
// NULL with *err set.
void* scratch_address(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cached[dev] = cus;
  return cus;
}

}  // namespace

namespace gdn {

size_t prefill_split_workspace_bytes(int N, int T, int HQ, int HV) {
  if (N <= 0 || T < 0 || HQ <= 0 || HV <= 0) return 0;
  return seam_plan_offset(T / C + N, N, HQ, HV) + seam_bytes(N, T, HV);
}

int prefill_split_auto_slices(int N, int HV) {
  const long long chains = (long long)N * HV;
  const int cus = device_cu_count();
  if (chains <= 0 || cus <= 0) return 0;
  // 8 slices while they fit the CUs at once; 4 slices while they fit in two
  // rounds of one workgroup per CU (the longest chains first; measured faster
  // than one fused workgroup per chain at 128 chains on 256 CUs); past that
  // the fused kernel.
  if (chains * 8 <= cus) return 8;
  if (chains * 4 <= 2LL * cus) return 4;
  return 0;
}

bool prefill_split_slices_valid(int slices) { return slices == 4 || slices == 8; }

int device_cus() { return device_cu_count(); }

size_t prefill_scratch_bytes() { return kScratchBytes; }

void* prefill_scratch(hipError_t* err) { return scratch_address(err); }

int prefill_split_launch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* state,
                         const float* A_log, const uint16_t* a, const float* dt_bias,
                         const uint16_t* b, const void* cu_seqlens, int cu_is_int32, int N, int T,
                         int HQ, int HV, float scale, uint16_t* out, float* final_state,
                         int slices, void* workspace, int flags, hipStream_t st, uint16_t* h,
                         int h_chunks) {
  char* ws = static_cast<char*>(workspace);
  const bool l2 = (flags & GDN_QK_L2NORM) != 0;
  const bool no_seams = (flags & GDN_NO_SEAMS) != 0;
  if (cu_is_int32) {
    const int32_t* cu = static_cast<const int32_t*>(cu_seqlens);
    return l2 ? launch_split_t<int32_t, true>(q, k, v, state, A_log, a, dt_bias, b, cu, N, T, HQ, HV, scale,
                                              out, final_state, slices, ws, h, h_chunks, no_seams, st)
              : launch_split_t<int32_t, false>(q, k, v, state, A_log, a, dt_bias, b, cu, N, T, HQ, HV, scale,
                                               out, final_state, slices, ws, h, h_chunks, no_seams, st);
  }
  const int64_t* cu = static_cast<const int64_t*>(cu_seqlens);
  return l2 ? launch_split_t<int64_t, true>(q, k, v, state, A_log, a, dt_bias, b, cu, N, T, HQ, HV, scale,
                                            out, final_state, slices, ws, h, h_chunks, no_seams, st)
            : launch_split_t<int64_t, false>(q, k, v, state, A_log, a, dt_bias, b, cu, N, T, HQ, HV, scale,
                                             out, final_state, slices, ws, h, h_chunks, no_seams, st);
}

}  // namespace gdn
