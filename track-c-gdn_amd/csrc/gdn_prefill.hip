// GDN chunked varlen prefill (gfx950 / CDNA4, wave64, MFMA).
//
// Replaces the reference prefill pipeline (five Triton launches plus host
// metadata; gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py
// :1570-1633, 1728-1759, 1762-1802) by one launch: a workgroup owns one
// (sequence, v-head) chain and walks its 64-token chunks in order, gates
// included.  The fp32 state S [V=128, K=128] never leaves registers between
// chunks, and nothing but q/k/v/a/b is read and o / final state written (and,
// in the kH instantiation, the state entering every chunk).
//
// Per chunk (C = 64 rows, gam = chunk-local cumsum of the log-decay,
// S = state at chunk start), the same mathematics as the reference
// (kernel.py:509-525, 661-796, 1153-1339, 1447-1496) arranged so that W and U
// are never formed:
//   A   = tril_strict(beta_i e^{gam_i-gam_j} K K^T)      (bf16 MFMA, exact products)
//   P   = scale tril_incl(e^{gam_i-gam_j} Q K^T)          (bf16 MFMA, exact products)
//   Tm  = (I + A)^-1      (fp32 16x16 diagonal blocks by substitution, MFMA block merges)
//   X   = diag(beta) (V - diag(e^gam) K S^T)
//   Vn  = Tm X          ( = U - W S^T of the reference )
//   O   = scale diag(e^gam) Q S^T + P Vn
//   S  <- e^{gam_L} S + (diag(e^{gam_L-gam}) Vn)^T K
// The products on the state's path (K S^T, Tm X, the S update) run on fp16
// operands (bf16 inputs convert exactly in fp16's normal range; fp16 keeps 3
// more mantissa bits than bf16 for the state and intermediates); Q S^T, which
// only reaches the bf16 output, takes the raw bf16 Q rows and a bf16 copy of
// S.  All products accumulate in fp32.
//
// Chain wave w (of 4) owns state rows v in [32w, 32w+32), two 16-row column
// tiles: every product that touches S, X, Vn or O is split along v, so the
// chain waves never exchange state.  Four preparation waves build the next
// chunk's A, Tm, P, gates and LDS copies alongside.
// The state lives as S^T accumulator tiles of 16x16x32 MFMAs; because an MFMA
// reduces over an arbitrary pairing of its k-slots, two stacked accumulator
// tiles are used directly as the B operand of the next product (k-slot e of
// lane group q is row 16(e/4) + 4q + e%4), with the A operand read from LDS in
// the matching order (the p32 column order below): no cross-lane shuffles,
// only fp32->fp16 packs.

#include "gdn_prefill_common.h"
#include "gdn_prefill_split.h"
#include "../../include/gdn_hip.h"

#include <algorithm>
#include <cstring>
#include <functional>
#include <queue>
#include <vector>

namespace {

using namespace gdn;

constexpr int kChainWaves = 4;              // state-chain waves, one per SIMD, 32 state rows each
constexpr int kPrepWaves = 4;               // preparation / copy waves, one per SIMD
constexpr int kWaves = kChainWaves + kPrepWaves;
constexpr int kThreads = kWaves * 64;
constexpr int kPrepThreads = kPrepWaves * 64;
constexpr int kRowsPerWave = D / kChainWaves;   // state rows (v) per chain wave
constexpr int kTiles = kRowsPerWave / 16;        // 16-row column tiles per chain wave

// The state chain.  One workgroup of 8 waves per (sequence, v-head), two on
// each SIMD: waves 0-3 run the chain (wave w owns state rows v in
// [32w, 32w+32), two 16-row column tiles; all of its products are 16x16x32
// MFMAs) and store the outputs; waves 4-7 (preparation waves 0-3) prepare
// chunks and issue every copy into LDS.  In iteration i the chain works on
// chunk i while the preparation waves build chunk i+1, in four phases
// separated by LDS barriers:
//   P1   chain : X = beta (V - e^gam K S^T) prep : 16-row merges of Tm_i (prep waves 2, 3);
//                                                  rest of P_i; gate data of chunk i+1
//                                                  (prep wave 0)
//   P2   chain : Vn = Tm X, Vd,             prep : copy of V_{i+1}; A_{i+1} tiles of
//                scale e^gam Q S^T                 the diagonal 32-row blocks
//   P3a  chain : O = scale e^gam Q S^T      prep : rows 0-11 of the Tm_{i+1} diagonal
//                + P Vn -> HBM; S update,          blocks (prep wave 0); lower-left
//                first half of k                   A_{i+1} tiles; fp16 K_{i+1}
//   P3b  chain : S update, second half;     prep : rows 12-15 of those blocks (prep
//                K S^T of chunk i+1                wave 0); P_{i+1} tiles; copies of
//                                                  K/Q of chunk i+2
// The 32-row merge of Tm is left to the chain: Vn = Tm X is applied as
// Vn_top = T_a X_top, Vn_bot = T_b (X_bot - A_ba Vn_top).
// Raw K and Q rows are double-buffered by chunk parity, so the chain reads the
// Q rows of chunk i while the P tiles of chunk i+1 read the next ones.  The S
// update reads K^T through transposing LDS reads.  Copies are issued one
// phase or more before their first use and waited for with explicit vmcnt
// counts by the waves that issued them.  The chain reads the operands of a
// phase at the end of the phase before whenever no wave overwrites them in
// between, and its barriers leave those reads in flight.  Which wave computes
// which tile is fixed at compile time, so tile offsets are immediates.
//
// kL2 (option GDN_QK_L2NORM): the q and k rows are used L2-normalised.  The
// copying waves compute each row's factor (sum x^2 + 1e-6)^(-1/2) from the
// rows they copied, right after their wait for them, and the factors scale
// the products: the fp16 K rows (so K S^T and the state update see k-hat),
// the A and P tiles (row and column factors) and the e^gam factor of S Q^T.
//
// kH: the state entering every chunk is also written, bf16, to
// hout[chunk_offset(n) + ch][hv][v][k] (chunk_offset(n) = the chunks of the
// sequences before n), skipping slots at or past h_chunks.  The values are
// the bf16 fragments the chain forms anyway for S Q^T.
// Slot swizzle of the raw V rows: 16-byte chunk c of row t sits in slot
// c ^ vsw(t).  The chain reads V with transposing 8-byte reads; a read cycle
// serves 8 rows with 4 lanes on 32 contiguous bytes (two slots) of each, and
// with vsw(t) = 2 (t % 8) + (t / 8) % 2 the 8 rows' slot pairs are distinct
// (with t % 16 two rows share each pair).
__device__ __forceinline__ int vsw(int t) { return ((t & 7) << 1) | ((t >> 3) & 1); }

// The seams of a fused launch (time splits of the longest chains, run on the
// CUs that shorter chains leave idle; the algebra is stated in
// gdn_prefill_common.h), planned on the host from the sequence lengths and
// passed by value.  Seam j cuts sequence seq[j] (of host bounds bos[j],
// len[j]) at chunk sp[j]: its G v-heads' head chains run in the chains' grid
// and stop at the cut; its tail chains (zero state, then transition) run in
// extra workgroups from base_ids on.  OX rows of seam j start at ox_row[j].
struct FusedSeams {
  int count;                // 0 .. kMaxSeams
  int base_ids;             // workgroup ids of the chains' grid
  int seq[kMaxSeams];
  int sp[kMaxSeams];
  int bos[kMaxSeams];
  int len[kMaxSeams];
  int ox_row[kMaxSeams];
  char* region;             // seam region of count slots
};

// One zero V row: the transition chains copy it in place of their V rows
// (row offsets dropped), so their copies and waits are the chain's own.
__device__ __align__(256) uint16_t g_zero_v_row[D];

template <typename CuT, bool kL2, bool kH>
__global__ __launch_bounds__(kThreads, 1) void gdn_prefill_chain_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ h0,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    const CuT* __restrict__ cu_seqlens, int N, int T, int HQ, int HV,
    float scale, uint16_t* __restrict__ out, float* __restrict__ ht,
    uint16_t* __restrict__ hout, int h_chunks, const FusedSeams seams) {
  __shared__ Smem sm;
  __shared__ SmemRaw raw;
  __shared__ __align__(16) uint16_t rawV[C * D];     // V chunk (bf16, swizzled), DMA target
  __shared__ __align__(16) float gbuf[2][GSZ];       // gate data, DMA target, double-buffered
  // L2-norm factors of the K / Q rows of the chunks of parity 0 / 1 (kL2 only)
  __shared__ __align__(16) float nrm[kL2 ? 2 * 2 * C : 4];
  auto nk = [&](int pb) { return &nrm[(2 * pb + 0) * C]; };
  auto nq = [&](int pb) { return &nrm[(2 * pb + 1) * C]; };

  // Workgroup -> (sequence n, v-head hv).  The G = HV/HQ v-heads that share a
  // qk-head read the same K/Q rows; they get workgroup ids 8 apart, which the
  // dispatcher places on the same XCD (ids go round-robin over the 8 XCDs),
  // so the second read of a K/Q row can hit that XCD's L2.  Unit u = (n, hq)
  // and member m map to id 8 (G (u / 8) + m) + u % 8; ids past the last unit
  // exit at once.  Seams: the ids from seams.base_ids on take seam units
  // (seam j, hq) the same way, 2 G members each (G zero-state tails, then G
  // transition chains); the dispatcher starts them, seam by seam, as CUs free.
  // role 0: a whole chain; 1: a seam's head; 2: its zero-state tail; 3: its
  // transition chain.
  const int heads_per_qk = HV / HQ;
  int n, hq, hv, role = 0, sj = 0;
  if (seams.count == 0 || int(blockIdx.x) < seams.base_ids) {
    const int xcd = blockIdx.x & 7, id_row = blockIdx.x >> 3;
    const int unit = 8 * (id_row / heads_per_qk) + xcd;
    if (unit >= N * HQ) return;
    n = unit / HQ;
    hq = unit - n * HQ;
    hv = hq * heads_per_qk + (id_row - (id_row / heads_per_qk) * heads_per_qk);
#pragma unroll
    for (int j = 0; j < kMaxSeams; ++j)
      if (j < seams.count && seams.seq[j] == n) {
        role = 1;
        sj = j;
      }
  } else {
    const int e = int(blockIdx.x) - seams.base_ids;
    const int xcd = e & 7, id_row = e >> 3;
    const int su = 8 * (id_row / (2 * heads_per_qk)) + xcd;
    if (su >= seams.count * HQ) return;
    const int w = id_row - (id_row / (2 * heads_per_qk)) * (2 * heads_per_qk);
    sj = su / HQ;
    hq = su - sj * HQ;
    role = 2 + w / heads_per_qk;
    hv = hq * heads_per_qk + w % heads_per_qk;
    n = 0;
#pragma unroll
    for (int j = 0; j < kMaxSeams; ++j)
      if (j == sj) n = seams.seq[j];
  }
  int sp_j = 0, ox_row_j = 0, tail_j = 0;   // this seam's cut, first OX row, tail tokens
#pragma unroll
  for (int j = 0; j < kMaxSeams; ++j)
    if (role != 0 && j == sj) {
      sp_j = seams.sp[j];
      ox_row_j = seams.ox_row[j];
      tail_j = seams.len[j] - C * seams.sp[j];
    }
  int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: keep it scalar
  int lane = tid & 63;
  int g = lane >> 4;              // lane group (16x16 MFMA layouts)
  int c = lane & 15;
  const bool is_chain = wave < kChainWaves;
  const int pw = wave - kChainWaves;          // preparation wave index (valid when !is_chain)
  int ptid = tid - kChainWaves * 64;          // preparation thread index
  const int v0 = kRowsPerWave * (wave & (kChainWaves - 1));
  const int vrow = v0 + c;        // state row v owned by this lane (chain waves)
  // |scale| enters the P exponent and its sign the P product (scale < 0 is allowed)
  const float scale_l2 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(__log2f(fabsf(scale)))));
  const bool neg_scale = scale < 0.f;

  int bos, len;
  seq_bounds(cu_seqlens, n, T, bos, len);
  // A seam's head and tails run as sequences of their own: chunks [0, sp) and
  // [sp, ...), the tails' tokens clamped to the plan's (so a transition
  // chain's OX rows stay inside the region).
  if (role == 1) {
    len = min(len, C * sp_j);
  } else if (role >= 2) {
    const int cut = min(len, C * sp_j);
    bos += cut;
    len = max(0, min(len - cut, tail_j));
  }
  if (blockIdx.x == 0 && tid == 0) {
    // the plan of the seam pass
    int* plan = reinterpret_cast<int*>(seams.region);
#pragma unroll
    for (int j = 0; j < kMaxSeams; ++j)
      if (j < seams.count) {
        int* e = plan + kSeamPlanStride * j;
        e[SP_SEQ] = seams.seq[j];
        e[SP_BOS] = seams.bos[j];
        e[SP_LEN] = seams.len[j];
        e[SP_SPLIT] = seams.sp[j];
        e[SP_CHUNKS] = (seams.len[j] + C - 1) / C;
        e[SP_OX_ROW] = seams.ox_row[j];
      }
  }
  // gate inputs of this head (uniform)
  const float a_log_exp = expf(A_log[hv]);
  const float dtb = dt_bias[hv];
  uint16_t ga = 0, gb = 0;          // a, b of token (chunk start + lane), preparation wave 0
  const size_t qk_stride = size_t(HQ) * D;   // elements per token in q / k
  const size_t v_stride = size_t(HV) * D;    // elements per token in v / out
  const int n_chunks = (len + C - 1) / C;
  int h_base = 0;                   // kH: chunks of the sequences before n
  if constexpr (kH) {
    int part = 0;                   // lanes take every 64th sequence, then a wave sum
    for (int m = lane; m < n; m += 64) {
      int bm, lm;
      seq_bounds(cu_seqlens, m, T, bm, lm);
      part += (lm + C - 1) / C;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
    h_base = __builtin_amdgcn_readfirstlane(part);
  }
  auto chunk_len = [&](int ch) { return min(C, len - ch * C); };

  // Upper 16x16 tiles inside the diagonal 32x32 blocks of Tm / P are read by
  // the products and must be zero; they are never written afterwards.
  for (int e = tid; e < 2 * 16 * 16; e += kThreads) {
    const int blk = e >> 8, r = (e >> 4) & 15, cc = e & 15;
    const int R = 32 * blk + r, pc = p32(32 * blk + 16 + cc);
    sm.Tm[R * TLD + pc] = (_Float16)0.f;
    sm.P[R * TLD + pc] = (_Float16)0.f;
  }

  // ---------------- copies into LDS (preparation waves 1-3).  An instruction
  // covers 4 rows: lane l carries row row0 + l/16, swizzle slot l%16 (rows past
  // the chunk end are clamped to its last row).  The 16 groups of 4 rows go
  // 6 / 5 / 5 to waves 1 / 2 / 3, one instruction per group and copy.
  // Preparation wave 0 issues no copies, only its loads of a and b, so the
  // waits the compiler places for those count nothing else.
  constexpr int kMaxGroups = 6;
  const int n_groups = (is_chain || pw == 0) ? 0 : (pw == 1 ? 6 : 5);
  const int group0 = pw == 1 ? 0 : (pw == 2 ? 6 : 11);
  auto group_row0 = [&](int j) { return 4 * (group0 + j); };
  // Byte offsets, from a chunk's first row, of the 16 bytes this lane copies
  // in group j, for q / k and for v: fixed per lane, so full chunks copy from
  // a uniform base with no per-copy address arithmetic.
  uint32_t dma_qk[kMaxGroups], dma_v[kMaxGroups];
#pragma unroll
  for (int j = 0; j < kMaxGroups; ++j) {
    const int row = group_row0(j) + (lane >> 4);
    dma_qk[j] = uint32_t(row) * uint32_t(qk_stride * 2) + uint32_t((lane & 15) ^ (row & 15)) * 16u;
    dma_v[j] = (role == 3 ? 0u : uint32_t(row) * uint32_t(v_stride * 2)) + uint32_t((lane & 15) ^ vsw(row)) * 16u;
  }
  auto copy_rows = [&](const uint16_t* src, size_t stride, size_t col0, const uint32_t* offs, int ch,
                       uint16_t* dst, bool is_v) {
    const int t0 = bos + ch * C;
    const int L = chunk_len(ch);
    if (L == C) {
      const uint16_t* base = src + size_t(t0) * stride + col0;
#pragma unroll
      for (int j = 0; j < kMaxGroups; ++j)
        if (j < n_groups) lds_dma16_saddr(base, offs[j], &dst[group_row0(j) * D]);
    } else {
#pragma unroll
      for (int j = 0; j < kMaxGroups; ++j) {
        if (j < n_groups) {
          const int row0 = group_row0(j);
          const int row = row0 + (lane >> 4);
          const int src_chunk = (lane & 15) ^ (is_v ? vsw(row) : (row & 15));
          lds_dma16(src + size_t(t0 + min(row, L - 1)) * stride + col0 + 8 * src_chunk, &dst[row0 * D]);
        }
      }
    }
  };
  auto copy_k = [&](int ch) { copy_rows(k, qk_stride, size_t(hq) * D, dma_qk, ch, raw.k[ch & 1], false); };
  auto copy_q = [&](int ch) { copy_rows(q, qk_stride, size_t(hq) * D, dma_qk, ch, raw.q[ch & 1], false); };
  auto copy_kq = [&](int ch) { copy_k(ch); copy_q(ch); };
  // the transition chain copies the zero row for every V row
  const uint16_t* v_src = role == 3 ? g_zero_v_row : v;
  const size_t v_src_stride = role == 3 ? 0 : v_stride;
  const size_t v_src_col = role == 3 ? 0 : size_t(hv) * D;
  auto copy_v = [&](int ch) { copy_rows(v_src, v_src_stride, v_src_col, dma_v, ch, rawV, true); };
  // L2-norm factors of the 4 n_groups rows this wave copied into buf, from the
  // diagonal of their Gram matrix: two 16-row tiles, each one bf16 MFMA chain
  // with the same registers as both operands (squares exact, fp32 sums).  Tile
  // lane (g, c) supplies row c and holds Gram entries (4 g + e, c), so the
  // diagonal entry of row c sits in lane (c / 4, c), element c % 4.  Rows past
  // the wave's last repeat it.  Call after the wait for those copies.
  auto norm_rows = [&](const uint16_t* buf, float* dstf) {
    if (n_groups == 0) return;
    const int nrows = 4 * n_groups;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int i = min(16 * tt + c, nrows - 1);
      const int r = group_row0(0) + i;
      bf16x8_t f[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) f[ks] = ld16_bf(&buf[raw_off(r, 32 * ks + 8 * g)]);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc = mfma16_bf(f[ks], f[ks], acc);
      const float d = (c & 2) ? ((c & 1) ? acc[3] : acc[2]) : ((c & 1) ? acc[1] : acc[0]);
      if ((c >> 2) == g && 16 * tt + c < nrows) dstf[r] = l2norm_rsqrt(d);
    }
  };
  auto load_ab = [&](int ch) {      // a, b of the chunk's tokens for gate_compute (wave 0)
    const int L = chunk_len(ch);
    const size_t gi = size_t(bos + ch * C + min(lane, L - 1)) * HV + hv;
    ga = a[gi];
    gb = b[gi];
  };

  // Gate data of chunk ch (reference PRE:1706-1722 and the chunk-local cumsum
  // of PRE:1721) from a / b loaded by load_ab, into gbuf[ch & 1]: lane =
  // token; rows past the sequence end carry a zero log-decay and beta = 0.
  // Preparation wave 0.
  auto gate_compute = [&](int ch) {
    constexpr float kLog2e = 1.44269504088896341f, kLn2 = 0.69314718055994531f;
    const int L = chunk_len(ch);
    float ld = 0.f, bt = 0.f;
    if (lane < L) {
      // softplus(x) = max(x, 0) + ln(1 + e^-|x|); sigmoid(y) = 1 / (1 + e^-y)
      const float x = bf16_bits_to_f32(ga) + dtb;
      const float sp = fmaxf(x, 0.f) + kLn2 * __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e));
      ld = -a_log_exp * sp;
      bt = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-bf16_bits_to_f32(gb) * kLog2e));
    }
    ld = wave_inclusive_scan(ld);       // gam: chunk-local cumsum (<= 0)
    const float l2 = ld * kLog2e;
    const float gl2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l2), L - 1));
    const float eg = __builtin_amdgcn_exp2f(l2);
    float* gdst = gbuf[ch & 1];
    gdst[G_L2 + lane] = l2;
    gdst[G_BETA + lane] = bt;
    gdst[G_EG + lane] = eg;
    gdst[G_EGS + lane] = scale * eg;
    gdst[G_ED + lane] = __builtin_amdgcn_exp2f(gl2 - l2);
  };

  // ---------------- preparation steps (state-independent)
  // Raw bf16 K rows of chunk ch -> fp16 operand rows Kc[ch & 1] [t][p32(k)],
  // rows t >= L -> 0, by preparation waves 1-3: items ptid - 64 + 192 j,
  // j = 0..5, below 1024.  Item i fills the 16 bytes 8 s .. 8 s + 7 (p32
  // positions, s = i % 16) of row cv_row(i / 16): columns 32 (s / 4) + 4 (s % 4)
  // .. +3 and the same + 16, two 8-byte pieces of the raw row (16-byte slots
  // 2 apart, so the second offset is the first ^ 32 bytes).  cv_row swaps the
  // two low bits of the row index: a read cycle of 32 lanes covers rows r and
  // r + 2, whose swizzled slot sets are disjoint (rows r and r + 1 share
  // theirs), and every write is 16 bytes: no LDS bank conflicts either way.
  constexpr int kCvThreads = kPrepThreads - 64;
  constexpr int kCvItems = (C * (D / 8) + kCvThreads - 1) / kCvThreads;   // 6
  auto cv_row = [](int item) {
    const int r = item >> 4;
    return (r & ~3) | ((r & 1) << 1) | ((r >> 1) & 1);
  };
  uint32_t cv_src[kCvItems], cv_dst[kCvItems];    // byte offsets into a raw K buffer / a Kc buffer
#pragma unroll
  for (int j = 0; j < kCvItems; ++j) {
    const int item = (ptid - 64) + kCvThreads * j;
    const int row = cv_row(item), sl = item & 15;
    cv_src[j] = uint32_t(raw_off(row, 32 * (sl >> 2) + 4 * (sl & 3))) * 2u;
    cv_dst[j] = uint32_t(row * KCLD + 8 * sl) * 2u;
  }
  auto convert_k = [&](int ch) {
    const char* src = reinterpret_cast<const char*>(raw.k[ch & 1]);
    char* dst = reinterpret_cast<char*>(sm.Kc[ch & 1]);
    const int L = chunk_len(ch);
#pragma unroll
    for (int j = 0; j < kCvItems; ++j) {
      if (j == kCvItems - 1 && (ptid - 64) + kCvThreads * j >= C * (D / 8)) break;   // uniform per wave
      uint2 wa = *reinterpret_cast<const uint2*>(src + cv_src[j]);
      uint2 wb = *reinterpret_cast<const uint2*>(src + (cv_src[j] ^ 32u));
      if (L < C) {
        const uint32_t m = cv_row((ptid - 64) + kCvThreads * j) < L ? 0xffffffffu : 0u;
        wa.x &= m; wa.y &= m; wb.x &= m; wb.y &= m;
      }
      float f[8];
      unpack_bf16x2(wa.x, f[0], f[1]); unpack_bf16x2(wa.y, f[2], f[3]);
      unpack_bf16x2(wb.x, f[4], f[5]); unpack_bf16x2(wb.y, f[6], f[7]);
      if constexpr (kL2) {
        const float r = nk(ch & 1)[cv_row((ptid - 64) + kCvThreads * j)];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] *= r;
      }
      *reinterpret_cast<f16x8*>(dst + cv_dst[j]) =
          f16x8{(_Float16)f[0], (_Float16)f[1], (_Float16)f[2], (_Float16)f[3],
                (_Float16)f[4], (_Float16)f[5], (_Float16)f[6], (_Float16)f[7]};
    }
  };
  // Per-lane swizzled offsets of the 8-column pieces this lane reads from a
  // raw row r with r % 16 == c: piece 4 ks + g sits in slot (4 ks + g) ^ c.
  int raw_lane[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) raw_lane[ks] = c * D + 8 * ((4 * ks + g) ^ c);
  // A tile = tril_strict(beta_i e^{gam_i - gam_j} K K^T) from the raw bf16
  // rows (bf16 MFMA: the inputs are exact).  The product is formed transposed
  // (K_j K_i^T), so that lane (g, c) holds row 16 ti + c, columns 16 tj + 4 g
  // .. +3 of the tile: 4 adjacent entries, one store.  Diagonal tiles store
  // zeros above the diagonal.
  auto tile_A = [&](auto tile_c, const float* gd, int pb) {
    constexpr int ti = Tile16<decltype(tile_c)::value>::ti;
    constexpr int tj = Tile16<decltype(tile_c)::value>::tj;
    bf16x8_t fa[4], fb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      fa[ks] = ld16_bf(&raw.k[pb][raw_lane[ks] + 16 * ti * D]);
      fb[ks] = ld16_bf(&raw.k[pb][raw_lane[ks] + 16 * tj * D]);
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = mfma16_bf(fb[ks], fa[ks], acc);
    const float gr = gd[G_L2 + 16 * ti + c];
    float br = gd[G_BETA + 16 * ti + c];
    const f32x4 gcol = *reinterpret_cast<const f32x4*>(&gd[G_L2 + 16 * tj + 4 * g]);
    if constexpr (kL2) {
      br *= nk(pb)[16 * ti + c];
      acc *= *reinterpret_cast<const f32x4*>(&nk(pb)[16 * tj + 4 * g]);
    }
    f32x4 val;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      val[i] = br * __builtin_amdgcn_exp2f(gr - gcol[i]) * acc[i];
      if (ti == tj) val[i] = (c > 4 * g + i) ? val[i] : 0.f;
    }
    if (ti >= 2 && tj <= 1) {     // lower-left 32x32 block, negated: an MFMA operand of the chain
      *reinterpret_cast<f16x4_t*>(&sm.Aba[(16 * (ti - 2) + c) * BLD + 8 * g + 4 * tj]) =
          f16x4_t{(_Float16)-val[0], (_Float16)-val[1], (_Float16)-val[2], (_Float16)-val[3]};
    } else {
      *reinterpret_cast<f32x4*>(&sm.A[(16 * ti + c) * ALD + 16 * tj + 4 * g]) = val;
    }
  };
  // P tiles = scale tril_incl(e^{gam_i - gam_j} Q K^T) from the raw bf16 rows
  // (bf16 MFMA: the inputs are exact), formed transposed like the A tiles:
  // lane (g, c) holds row 16 ti + c, columns 16 tj + 4 g .. +3, which are 4
  // adjacent positions of the p32 order.  The tiles (ti, 2 s) and (ti, 2 s + 1)
  // are formed together (one set of Q fragments) and their 8 positions
  // 32 s + 8 g .. +7 go out as one 16-byte write; a tile above the diagonal is
  // written as zeros.  (Two 8-byte writes per lane down 16 rows of 160 bytes
  // meet in the LDS banks; one 16-byte write per lane does not.)  Rows past
  // the chunk end hold copies of its last row; they only reach output rows
  // that are never stored.
  auto tile_P_pair = [&](auto ti_c, auto s_c, const float* gd, int pb) {
    constexpr int ti = decltype(ti_c)::value;
    constexpr int tj0 = 2 * decltype(s_c)::value, tj1 = tj0 + 1;
    constexpr bool two = tj1 <= ti;
    bf16x8_t fa[4], fb0[4], fb1[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      fa[ks] = ld16_bf(&raw.q[pb][raw_lane[ks] + 16 * ti * D]);
      fb0[ks] = ld16_bf(&raw.k[pb][raw_lane[ks] + 16 * tj0 * D]);
      if constexpr (two) fb1[ks] = ld16_bf(&raw.k[pb][raw_lane[ks] + 16 * tj1 * D]);
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
      const float qn = nq(pb)[16 * ti + c];
      acc0 *= qn * *reinterpret_cast<const f32x4*>(&nk(pb)[16 * tj0 + 4 * g]);
      if constexpr (two) acc1 *= qn * *reinterpret_cast<const f32x4*>(&nk(pb)[16 * tj1 + 4 * g]);
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
    *reinterpret_cast<f16x8*>(&sm.P[(16 * ti + c) * TLD + 16 * tj0 + 8 * g]) = val;
  };
  // A tiles of the chunk of parity pb inside the diagonal 32-row blocks (the
  // inverse's input): 6 tiles over the 4 preparation waves.
  auto tiles_A = [&](const float* gd, int pb) {
    switch (pw) {
      case 0: tile_A(IC<0>{}, gd, pb); tile_A(IC<2>{}, gd, pb); break;
      case 1: tile_A(IC<5>{}, gd, pb); tile_A(IC<9>{}, gd, pb); break;
      case 2: tile_A(IC<1>{}, gd, pb); break;
      default: tile_A(IC<8>{}, gd, pb); break;
    }
  };
  // The lower-left 32x32 block (Aba, read by the chain): 4 tiles over
  // preparation waves 1-3, in a phase in which the chain does not read Aba.
  auto tiles_Aba = [&](const float* gd, int pb) {
    switch (pw) {
      case 0: tile_A(IC<4>{}, gd, pb); break;
      case 1: tile_A(IC<3>{}, gd, pb); break;
      case 2: tile_A(IC<6>{}, gd, pb); break;
      default: tile_A(IC<7>{}, gd, pb); break;
    }
  };
  // Rows [I0, I1) of the diagonal 16x16 blocks of Tm: lane group g inverts
  // block g by forward substitution in fp32 (lane = column); x holds the
  // solved rows, so a later call continues where an earlier one stopped.
  auto diag_rows = [&](auto i0_c, auto i1_c, float(&x)[16]) {
    constexpr int I0 = decltype(i0_c)::value, I1 = decltype(i1_c)::value;
    const float* Ab = &sm.A[(16 * g) * ALD + 16 * g];
    // Opaque copy of the column index: keeps the identity selects inside
    // the chunk loop instead of being hoisted into registers.
    int cid = c;
    asm volatile("" : "+v"(cid));
#pragma unroll
    for (int i = I0; i < I1; ++i) {   // the A rows of the whole range are read up front
      // two partial sums (alternate 4-column blocks) halve the dependent chain
      float s0 = (i == cid) ? 1.f : 0.f, s1 = 0.f;
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
      x[i] = i > 4 ? s0 + s1 : s0;
    }
    const int pc = p32(16 * g + c);
#pragma unroll
    for (int i = I0; i < I1; ++i) sm.Tm[(16 * g + i) * TLD + pc] = (_Float16)x[i];
  };
  // 16-row merge inside the 32-row block at a0: T_{a0+16.., a0..} = -T_22 A_21 T_11.
  auto merge16 = [&](int a0) {
    const f32x4 a4 = *reinterpret_cast<const f32x4*>(&sm.A[(a0 + 16 + c) * ALD + a0 + 4 * g]);
    const f16x4_t fa = {(_Float16)a4[0], (_Float16)a4[1], (_Float16)a4[2], (_Float16)a4[3]};
    f16x4_t fb;
    const int pcb = p32(a0 + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) fb[e] = sm.Tm[(a0 + 4 * g + e) * TLD + pcb];
    const f32x4 y = mfma16k16(fa, fb, f32x4{0.f, 0.f, 0.f, 0.f});
    const f16x4_t ft = *reinterpret_cast<const f16x4_t*>(&sm.Tm[(a0 + 16 + c) * TLD + p32(a0 + 16 + 4 * g)]);
    const f16x4_t fy = {(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
    const f32x4 t21 = mfma16k16(ft, fy, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int i = 0; i < 4; ++i) sm.Tm[(a0 + 16 + 4 * g + i) * TLD + pcb] = (_Float16)(-t21[i]);
  };
  // P tiles of the chunk of parity pb over preparation waves 1-3, in two
  // parts: 6 tiles after the chain's last read of the previous P (P3b of the
  // previous iteration), 4 in P1 of the chunk's own iteration.
  auto tiles_P1 = [&](const float* gd, int pb) {
    switch (pw) {
      case 1: tile_P_pair(IC<2>{}, IC<0>{}, gd, pb); break;    // (2, 0), (2, 1)
      case 2: tile_P_pair(IC<3>{}, IC<0>{}, gd, pb); break;    // (3, 0), (3, 1)
      case 3: tile_P_pair(IC<3>{}, IC<1>{}, gd, pb); break;    // (3, 2), (3, 3)
      default: break;
    }
  };
  auto tiles_P2 = [&](const float* gd, int pb) {
    switch (pw) {
      case 1: tile_P_pair(IC<1>{}, IC<0>{}, gd, pb); break;    // (1, 0), (1, 1)
      case 2: tile_P_pair(IC<0>{}, IC<0>{}, gd, pb); break;    // (0, 0)
      case 3: tile_P_pair(IC<2>{}, IC<1>{}, gd, pb); break;    // (2, 2)
      default: break;
    }
  };
  if (is_chain) {
    // ================= chain waves
    // output rows: out[bos + t], or a transition chain's OX rows
    uint16_t* out_rows = out;
    int out_row0 = bos;
    if (role == 3) {
      out_rows = reinterpret_cast<uint16_t*>(seams.region + seam_ox_offset(seams.count, HV));
      out_row0 = ox_row_j;
    }
    // Column tile u (0, 1) of this wave holds state rows v = v0 + 16 u + c.
    // initial state: Sacc[u][kb][i] = S[v0 + 16 u + c][16 kb + 4 g + i]
    f32x4 Sacc[kTiles][8];
#pragma unroll
    for (int u = 0; u < kTiles; ++u)
#pragma unroll
      for (int kb = 0; kb < 8; ++kb) Sacc[u][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (role == 3) {              // the transition chain starts from the identity
#pragma unroll
      for (int u = 0; u < kTiles; ++u)
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) Sacc[u][kb][i] = (vrow + 16 * u == 16 * kb + 4 * g + i) ? 1.f : 0.f;
    }
    if (h0 != nullptr && role < 2) {
      const float* src = h0 + (size_t(n) * HV + hv) * size_t(D) * D + size_t(vrow) * D;
#pragma unroll
      for (int u = 0; u < kTiles; ++u)
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
          Sacc[u][kb] = *reinterpret_cast<const f32x4*>(src + size_t(16 * u) * D + 16 * kb + 4 * g);
    }
    // kH: the bf16 fragments of column blocks 2 pp and 2 pp + 1 (s0, s1) of
    // the state entering chunk ch go to its h slot as whole 128-byte lines
    // (store_state_lines; lane (g, c) of tile u holds row v0 + 16 u + c).
    const uint32_t h_lane = state_lines_lane(g, c);
    auto store_h = [&](int ch, int pp, const bf16x8_t (&s0)[kTiles], const bf16x8_t (&s1)[kTiles]) {
      if constexpr (kH) {
        const int slot = h_base + ch;
        if (slot < h_chunks) {
          char* base = reinterpret_cast<char*>(hout) + (size_t(slot) * HV + hv) * size_t(D * D * 2) +
                       size_t(v0) * (D * 2) + 128 * pp;
#pragma unroll
          for (int u = 0; u < kTiles; ++u) store_state_lines(base + u * (16 * D * 2), h_lane, c, s0[u], s1[u]);
        }
      }
    };
    // KS[u] += K[:, 32 p0 .. 32 p0 + 63] S^T[32 p0 .., tile u] for the chunk whose
    // fp16 K rows are in Kc[kb_buf]; columns 0-63 use state entries k < 64,
    // updated in the first half of the state update.  The 8 K fragments are
    // read before the first product and serve both column tiles.
    f32x4 KS[kTiles][4];
    // K fragments of column blocks p0, p0 + 1 of Kc[kb_buf]: issued ahead of
    // their products (LDS reads wait behind the other waves' traffic).
    typedef f16x8 KFrag[2][4];
    auto load_kf = [&](int kb_buf, int p0, KFrag& kf) {
      const _Float16* kbase = &sm.Kc[kb_buf][c * KCLD + 8 * g];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) kf[p][tb] = ld16(kbase + 16 * tb * KCLD + 32 * (p0 + p));
    };
    auto mul_kf = [&](int p0, KFrag& kf) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        f16x8 sb[kTiles];
#pragma unroll
        for (int u = 0; u < kTiles; ++u) sb[u] = pack2(Sacc[u][2 * (p0 + p)], Sacc[u][2 * (p0 + p) + 1]);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          asm volatile("" : "+v"(kf[p][tb]));   // products wait here, not between the reads
#pragma unroll
          for (int u = 0; u < kTiles; ++u) KS[u][tb] = mfma16(kf[p][tb], sb[u], KS[u][tb]);
        }
      }
    };
    KFrag kf_lo, kf_hi;     // columns 0-63 / 64-127 of the next chunk's K
    auto zero_ks = [&]() {
#pragma unroll
      for (int u = 0; u < kTiles; ++u)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) KS[u][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    };
    if (n_chunks > 0) {           // prologue: the preparation waves build chunk 0
      lds_barrier();
      lds_barrier();
      zero_ks();
      load_kf(0, 0, kf_lo);
      load_kf(0, 2, kf_hi);
      asm volatile("" ::: "memory");
      mul_kf(0, kf_lo);
      mul_kf(2, kf_hi);
      lds_barrier();
    }
    for (int ch = 0; ch < n_chunks; ++ch) {
      const int L = chunk_len(ch);
      const int kb_buf = ch & 1;
      const float* gd = gbuf[ch & 1];

      // ---- P1: X = beta (V - e^gam K S^T) in place of KS; at the end, the A_ba
      //      tiles and the Q fragments of column block 0 are read for P2.
      {
        // V[16 tb + 4 g + i][v0 + 16 u + c], i = 0..3, by one transposing read per
        // (u, tb): lane 4 m + j of group g reads columns v0 + 16 u + 4 j .. +3 of
        // row 16 tb + 4 g + m (8 contiguous bytes of a swizzled 16-byte slot).
        i16x4_t vv[kTiles][4];
        {
          const int m = c >> 2, j = c & 3;
#pragma unroll
          for (int u = 0; u < kTiles; ++u) {
            const int col = v0 + 16 * u + 4 * j;
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
              const int t = 16 * tb + 4 * g + m;
              vv[u][tb] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (__attribute__((address_space(3))) i16x4_t*)&rawV[t * D + 8 * ((col >> 3) ^ vsw(t)) + (col & 7)]);
            }
          }
        }
        f32x4 eg[4], bt[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          eg[tb] = *reinterpret_cast<const f32x4*>(&gd[G_EG + 16 * tb + 4 * g]);
          bt[tb] = *reinterpret_cast<const f32x4*>(&gd[G_BETA + 16 * tb + 4 * g]);
        }
        // every read issued before the first use (the asm operands keep the
        // conversions of V below this point)
        asm volatile("" ::: "memory");
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) asm volatile("" : "+v"(vv[u][tb]));
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              KS[u][tb][i] = bt[tb][i] * (bf16_bits_to_f32(uint16_t(vv[u][tb][i])) - eg[tb][i] * KS[u][tb][i]);
        // X is formed here, so the V rows (overwritten in P2) have been read
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) asm volatile("" : "+v"(KS[u][tb]));
      }
      f16x8 ab[2];
      bf16x8_t qf[2][4];      // Q fragments of column blocks p, p + 1 (double-buffered)
      auto load_qf = [&](int p, bf16x8_t(&dst)[4]) {
        // Element offsets, in a raw Q row t with t % 16 == c, of the two
        // 4-column pieces lane group g feeds as k-slots 0-3 / 4-7 of the
        // MFMA over column block p: columns 32 p + 4 g .. +3 and
        // 32 p + 16 + 4 g .. +3, the order in which two stacked S^T
        // accumulator tiles give the B operand.
        const int sw = (g >> 1) ^ c;
        const uint16_t* qraw = &raw.q[kb_buf][c * D + 4 * (g & 1)];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const bf16x4_t lo = *reinterpret_cast<const bf16x4_t*>(&qraw[16 * tb * D + 8 * ((4 * p) ^ sw)]);
          const bf16x4_t hi = *reinterpret_cast<const bf16x4_t*>(&qraw[16 * tb * D + 8 * ((4 * p + 2) ^ sw)]);
          // keeps the two reads of one fragment next to each other: paired with
          // reads of other fragments they would land in registers that need moves
          asm volatile("" ::: "memory");
          dst[tb] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
      };
      {
#pragma unroll
        for (int j = 0; j < 2; ++j) ab[j] = ld16(&sm.Aba[(16 * j + c) * BLD + 8 * g]);
        load_qf(0, qf[0]);
      }
      lds_barrier_keep<15>();   // A_ba and Q stay untouched in P2

      // ---- P2: Vn = Tm X, Vd; scale e^gam Q S^T
      f16x8 Vdb[kTiles][2], Vnb[kTiles][2];
      {
        // Tm = [[T_a, 0], [-T_b A_ba T_a, T_b]] in 32-row blocks, so
        // Vn_top = T_a X_top and Vn_bot = T_b (X_bot - A_ba Vn_top).  The
        // operand tiles are read up front and serve both column tiles, whose
        // products are interleaved stage by stage; the preparation stores
        // -A_ba, so X_bot - A_ba Vn_top accumulates in the MFMA.
        f16x8 ta[2], tb2[2];
        f32x4 ed[4];            // e^{gam_L - gam} of this lane's rows, for Vd
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          ta[j] = ld16(&sm.Tm[(16 * j + c) * TLD + 8 * g]);
          tb2[j] = ld16(&sm.Tm[(16 * (j + 2) + c) * TLD + 32 + 8 * g]);
        }
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) ed[tb] = *reinterpret_cast<const f32x4*>(&gd[G_ED + 16 * tb + 4 * g]);
        load_qf(1, qf[1]);      // Q S^T operands of column block 1, used after Tm X
        asm volatile("" ::: "memory");
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        f32x4 Vn[kTiles][4];
        f16x8 xb[kTiles];
#pragma unroll
        for (int u = 0; u < kTiles; ++u) xb[u] = pack2(KS[u][0], KS[u][1]);
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) Vn[u][tb] = mfma16(ta[tb], xb[u], z);
#pragma unroll
        for (int u = 0; u < kTiles; ++u) Vnb[u][0] = pack2(Vn[u][0], Vn[u][1]);
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) KS[u][2 + tb] = mfma16(ab[tb], Vnb[u][0], KS[u][2 + tb]);
        // decayed copy for the state update: Vd = e^{gam_L - gam} Vn
#pragma unroll
        for (int u = 0; u < kTiles; ++u) Vdb[u][0] = pack2(Vn[u][0] * ed[0], Vn[u][1] * ed[1]);
#pragma unroll
        for (int u = 0; u < kTiles; ++u) xb[u] = pack2(KS[u][2], KS[u][3]);
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
          for (int tb = 2; tb < 4; ++tb) Vn[u][tb] = mfma16(tb2[tb - 2], xb[u], z);
#pragma unroll
        for (int u = 0; u < kTiles; ++u) {
          Vnb[u][1] = pack2(Vn[u][2], Vn[u][3]);
          Vdb[u][1] = pack2(Vn[u][2] * ed[2], Vn[u][3] * ed[3]);
        }
        // Tm and A_ba (overwritten in P3a) have been read once Vn and Vd exist
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
          for (int j = 0; j < 2; ++j) asm volatile("" : "+v"(Vnb[u][j]), "+v"(Vdb[u][j]));
      }
      // The output tiles are formed transposed, O^T = S Q^T + Vn^T P^T: lane
      // (g, c) of OT[u][tb] holds token 16 tb + c, state rows (output columns)
      // v0 + 16 u + 4 g .. +3, 8 contiguous bytes of an output row.  The
      // operand registers are those of the untransposed products, swapped.
      f32x4 OT[kTiles][4];
#pragma unroll
      for (int u = 0; u < kTiles; ++u)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) OT[u][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
      f16x8 pf[6];              // P tiles (t-block, k-block): 00 10 20 21 30 31, read for P3a
      f16x8 fa[2][2];           // K^T fragments of k-blocks 0, 1, read for P3a
      auto load_fa = [&](int kb0, f16x8(&dst)[2][2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int kq = p32(16 * (kb0 + j) + 4 * (c & 3));    // this lane's quad of columns
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const int tr0 = 32 * p + 4 * g + (c >> 2);
            const f16x4_t lo = ld_tr16(&sm.Kc[kb_buf][tr0 * KCLD + kq]);
            const f16x4_t hi = ld_tr16(&sm.Kc[kb_buf][(tr0 + 16) * KCLD + kq]);
            dst[j][p] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          }
        }
      };
      {
        // Column blocks 0, 1 of S Q^T here, blocks 2, 3 in P3a (their Q fragments
        // read here, before other chain waves stage outputs in the raw Q buffer)
        bf16x8_t sbh[kTiles];     // kH: block 0's fragments, stored with block 1's
#pragma unroll
        for (int p = 0; p < 2; ++p) {     // the 8 products of block p, then the reads of block p + 2
          bf16x8_t sb[kTiles];
#pragma unroll
          for (int u = 0; u < kTiles; ++u) sb[u] = pack2_bf(Sacc[u][2 * p], Sacc[u][2 * p + 1]);
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            asm volatile("" : "+v"(qf[p & 1][tb]));
#pragma unroll
            for (int u = 0; u < kTiles; ++u) OT[u][tb] = mfma16_bf(sb[u], qf[p & 1][tb], OT[u][tb]);
          }
          if (p == 0) {
#pragma unroll
            for (int u = 0; u < kTiles; ++u) sbh[u] = sb[u];
          } else {
            store_h(ch, 0, sbh, sb);
          }
          load_qf(p + 2, qf[p & 1]);
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int tb = 0, j = 0; tb < 4; ++tb)
#pragma unroll
          for (int p = 0; p <= (tb >> 1); ++p, ++j) pf[j] = ld16(&sm.P[(16 * tb + c) * TLD + 8 * g + 32 * p]);
        load_fa(0, fa);
      }
      const float egL = gd[G_EG + L - 1];
      lds_barrier_keep<15>();   // P, K and the gate data stay untouched in P3a

      // ---- P3a / P3b: state update, S = e^{gam_L} S + K^T Vd, in two halves of
      //      k.  Before it, in P3a, O = scale e^gam Q S^T + P Vn goes to HBM;
      //      after it, in P3b, K S^T of chunk ch+1.
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        if (half == 0) {
          bf16x8_t sbh[kTiles];   // kH: block 2's fragments, stored with block 3's
#pragma unroll
          for (int p = 2; p < 4; ++p) {   // the rest of S Q^T (S before this chunk's update)
            bf16x8_t sb[kTiles];
#pragma unroll
            for (int u = 0; u < kTiles; ++u) sb[u] = pack2_bf(Sacc[u][2 * p], Sacc[u][2 * p + 1]);
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
              asm volatile("" : "+v"(qf[p & 1][tb]));
#pragma unroll
              for (int u = 0; u < kTiles; ++u) OT[u][tb] = mfma16_bf(sb[u], qf[p & 1][tb], OT[u][tb]);
            }
            if (p == 2) {
#pragma unroll
              for (int u = 0; u < kTiles; ++u) sbh[u] = sb[u];
            } else {
              store_h(ch, 1, sbh, sb);
            }
          }
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            float egs = gd[G_EGS + 16 * tb + c];    // scale e^gam of this lane's token
            if constexpr (kL2) egs *= nq(kb_buf)[16 * tb + c];
#pragma unroll
            for (int u = 0; u < kTiles; ++u) OT[u][tb] *= egs;
          }
#pragma unroll
          for (int tb = 0, j = 0; tb < 4; ++tb)
#pragma unroll
            for (int p = 0; p <= (tb >> 1); ++p, ++j) {
              asm volatile("" : "+v"(pf[j]));
#pragma unroll
              for (int u = 0; u < kTiles; ++u) OT[u][tb] = mfma16(Vnb[u][p], pf[j], OT[u][tb]);
            }
          // P (overwritten in P3b) has been read once O exists
#pragma unroll
          for (int u = 0; u < kTiles; ++u)
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) asm volatile("" : "+v"(OT[u][tb]));
          // The chunk's output tile is staged in the raw Q buffer of this chunk
          // (last read in P2; the Q copy of chunk ch+2 goes there in P1 of the
          // next iteration), in the raw row layout; P3b stores whole rows from
          // it.  Lane (g, c) holds columns v0 + 16 u + 4 g .. +3 of token
          // 16 tb + c in tile u; v_permlane16_swap trades tile 1 of the even
          // 16-lane rows for tile 0 of the odd rows, which leaves the lane 8
          // adjacent columns v0 + 16 (g % 2) + 8 (g / 2) .. +7 (tile g % 2): one
          // 16-byte write, where two 8-byte writes down 16 rows meet in the
          // LDS banks.
          static_assert(kTiles == 2, "two column tiles per chain wave");
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const uint32_t a0 = cvt_pk_bf16(OT[0][tb][0], OT[0][tb][1]), a1 = cvt_pk_bf16(OT[0][tb][2], OT[0][tb][3]);
            const uint32_t b0 = cvt_pk_bf16(OT[1][tb][0], OT[1][tb][1]), b1 = cvt_pk_bf16(OT[1][tb][2], OT[1][tb][3]);
            const auto s0 = __builtin_amdgcn_permlane16_swap(a0, b0, false, false);
            const auto s1 = __builtin_amdgcn_permlane16_swap(a1, b1, false, false);
            *reinterpret_cast<u32x4_t*>(&raw.q[kb_buf][raw_off(16 * tb + c, v0 + 16 * (g & 1) + 8 * (g >> 1))]) =
                u32x4_t{s0[0], s1[0], s0[1], s1[1]};
          }
          asm volatile("" ::: "memory");
        }
        if (half == 1) {
          // Rows kOutRows w .. kOutRows (w + 1) - 1 of the staged output tile
          // (w = this chain wave), 4 rows per instruction, to HBM as whole
          // 256-byte rows.  All reads first, then the stores: one LDS round
          // trip instead of one per store.
          constexpr int kOutRows = C / kChainWaves;
          const size_t row_bytes = v_stride * sizeof(uint16_t);
          char* obase = reinterpret_cast<char*>(out_rows + size_t(out_row0 + ch * C) * v_stride + size_t(hv) * D);
          u32x4_t od[kOutRows / 4];
#pragma unroll
          for (int q4 = 0; q4 < kOutRows / 4; ++q4) {
            const int row = kOutRows * (v0 / kRowsPerWave) + 4 * q4 + (lane >> 4);
            od[q4] = *reinterpret_cast<const u32x4_t*>(&raw.q[kb_buf][raw_off(row, 8 * c)]);
          }
#pragma unroll
          for (int q4 = 0; q4 < kOutRows / 4; ++q4) {
            const int row = kOutRows * (v0 / kRowsPerWave) + 4 * q4 + (lane >> 4);
            if (L == C || row < L) store_b128_saddr(obase, uint32_t(row) * uint32_t(row_bytes) + uint32_t(16 * c), od[q4]);
          }
        }
        // K^T fragments of the next k-block pair are read before the products of
        // this pair (the first pair was read in P2, the third at the end of P3a)
#pragma unroll
        for (int kb0 = 4 * half; kb0 < 4 * half + 4; kb0 += 2) {
          f16x8 fn[2][2];
          if (kb0 + 2 < 8 && kb0 != 2) load_fa(kb0 + 2, fn);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int u = 0; u < kTiles; ++u) Sacc[u][kb0 + j] *= egL;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              asm volatile("" : "+v"(fa[j][p]));
#pragma unroll
              for (int u = 0; u < kTiles; ++u) Sacc[u][kb0 + j] = mfma16(fa[j][p], Vdb[u][p], Sacc[u][kb0 + j]);
            }
          }
          if (kb0 == 2) load_fa(4, fa);     // for P3b
          else if (kb0 + 2 < 8) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
              for (int p = 0; p < 2; ++p) fa[j][p] = fn[j][p];
          }
        }
        if (half == 1) {    // after the last chunk this reads stale rows and is never used
          zero_ks();
          load_kf(kb_buf ^ 1, 0, kf_lo);
          load_kf(kb_buf ^ 1, 2, kf_hi);
          asm volatile("" ::: "memory");
          mul_kf(0, kf_lo);
          mul_kf(2, kf_hi);
        }
        // K (both buffers) stays untouched in P3b and P1; the staged output
        // tile written in P3a is older than the 8 reads that may stay in flight
        if (half == 0) lds_barrier_keep<8>();
        else lds_barrier_keep<15>();
      }
    }
    asm volatile("" : "+v"(g), "+v"(c));
    if (role == 3) {
      // X stored transposed: X^T[k][v] = Sacc[u][kb][i] at k = 16 kb + 4 g + i, v = vrow + 16 u
      float* dst = reinterpret_cast<float*>(seams.region + seam_state_offset(HV, sj, hv, 2));
#pragma unroll
      for (int u = 0; u < kTiles; ++u)
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[size_t(16 * kb + 4 * g + i) * D + vrow + 16 * u] = Sacc[u][kb][i];
    } else {
      float* dst = (role == 0 ? ht + (size_t(n) * HV + hv) * size_t(D) * D
                              : reinterpret_cast<float*>(seams.region + seam_state_offset(HV, sj, hv, role - 1))) +
                   size_t(v0 + c) * D;
#pragma unroll
      for (int u = 0; u < kTiles; ++u)
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
          *reinterpret_cast<f32x4*>(dst + size_t(16 * u) * D + 16 * kb + 4 * g) = Sacc[u][kb];
    }
  } else {
    // ================= preparation waves
    // The preparation waves run single-wave dependency chains (Tm inverse and
    // merges, gates) that bound the chunk period; issuing their instructions
    // ahead of the chain waves' shortens it.
    __builtin_amdgcn_s_setprio(2);
    float dx[16];                 // solved rows of the Tm diagonal blocks (preparation wave 0)
    if (n_chunks > 0) {           // prologue: chunk 0 copied and prepared up to its Tm merges
      copy_kq(0);
      copy_v(0);
      if (pw == 0) load_ab(0);
      wait_vm<0>();
      if constexpr (kL2) {
        norm_rows(raw.k[0], nk(0));
        norm_rows(raw.q[0], nq(0));
      }
      if (pw == 0) {
        gate_compute(0);
        if (n_chunks > 1) load_ab(1);
      }
      if (n_chunks > 1) copy_k(1);   // Q of chunk 1 is copied in P1 of chunk 0
      lds_barrier();
      tiles_A(gbuf[0], 0);
      tiles_Aba(gbuf[0], 0);
      if (pw > 0) convert_k(0);
      lds_barrier();
      if (pw == 0) {
        diag_rows(IC<0>{}, IC<12>{}, dx);
        diag_rows(IC<12>{}, IC<16>{}, dx);
      } else {
        tiles_P1(gbuf[0], 0);
      }
      lds_barrier();
    }
    for (int ch = 0; ch < n_chunks; ++ch) {
      asm volatile("" : "+v"(tid), "+v"(lane), "+v"(g), "+v"(c), "+v"(ptid));
      const int nb = (ch + 1) & 1;          // parity of chunk ch+1
      const bool more = ch + 1 < n_chunks;
      // ---- P1: 16-row Tm merges of chunk ch (prep waves 2, 3); K rows of chunk
      //      ch+1 landed (copied in P2 of ch-1); gate data of ch+1 from a and b
      //      loaded in P1 of ch-1, then the loads of a and b of ch+2 (prep wave 0)
      if (pw >= kPrepWaves - 2) merge16(32 * (pw - (kPrepWaves - 2)));
      tiles_P2(gbuf[ch & 1], ch & 1);   // the rest of P of chunk ch (read by the chain in P3a)
      // Q rows of chunk ch+1 into the raw buffer of chunk ch-1 (its output tile
      // was stored from there in P3b), first read in P3b
      if (more) copy_q(ch + 1);
      if (more) {
        if (pw == 1) wait_vm<6>(); else wait_vm<5>();   // K of ch+1 landed; its Q copies may remain
        if constexpr (kL2) norm_rows(raw.k[nb], nk(nb));
        if (pw == 0) {
          gate_compute(ch + 1);
          if (ch + 2 < n_chunks) load_ab(ch + 2);
        }
      }
      lds_barrier();
      // ---- P2: V copy and the A tiles of the diagonal 32-row blocks of chunk ch+1
      if (more) {
        copy_v(ch + 1);           // every chain wave has read V of chunk ch
        tiles_A(gbuf[nb], nb);
      }
      if (ch + 2 < n_chunks) copy_k(ch + 2);   // raw K of chunk ch was last read in P1
      lds_barrier();
      // ---- P3a: rows 0-11 of the Tm diagonal blocks (prep wave 0), the lower-left
      //      A tiles and the fp16 K rows (prep waves 1-3) of chunk ch+1; the chain has
      //      read Aba of ch in P1 and Tm of ch in P2
      if (more) {
        if (pw == 0) diag_rows(IC<0>{}, IC<12>{}, dx);
        else convert_k(ch + 1);
        // Q of chunk ch+1 landed (read from P3b on); the V and K copies issued
        // in P2 may remain
        if (ch + 2 < n_chunks) {
          if (pw == 1) wait_vm<12>(); else wait_vm<10>();
        } else {
          if (pw == 1) wait_vm<6>(); else wait_vm<5>();
        }
        if constexpr (kL2) norm_rows(raw.q[nb], nq(nb));
      }
      lds_barrier();
      // ---- P3b: rows 12-15 of the Tm diagonal blocks (prep wave 0) and the P tiles
      //      (prep waves 1-3) of chunk ch+1, the chain having read P of ch in P3a;
      //      copies of chunk ch+2 into the raw buffers of ch; V of chunk ch+1
      //      landed (only the new K/Q copies, 12 on prep wave 1 and 10 on prep
      //      waves 2 and 3, remain outstanding)
      if (more) {
        tiles_Aba(gbuf[nb], nb);     // the chain read Aba of chunk ch by P2
        if (pw == 0) diag_rows(IC<12>{}, IC<16>{}, dx);
        else tiles_P1(gbuf[nb], nb);
      }
      if (ch + 2 < n_chunks) {
        if (pw == 1) wait_vm<6>(); else wait_vm<5>();   // the K copies of chunk ch+2 may remain
      } else if (more) {
        wait_vm<0>();
      }
      lds_barrier();
    }
  }
}

int check_prefill_args(const void* q, const void* k, const void* v, const void* A_log,
                       const void* a, const void* dt_bias, const void* b, const void* cu,
                       const void* out, const void* final_state, int N, int T, int HQ, int HV) {
  if (N < 0 || T < 0 || HQ <= 0 || HV <= 0 || HV % HQ != 0) return GDN_ERR_SHAPE;
  // Empty tensors may have no storage: token arrays are only needed when
  // T > 0, per-sequence arrays when N > 0 (a batch of empty sequences still
  // copies its initial states to the final states).
  if (!cu) return GDN_ERR_NULL;
  if (N > 0 && (!A_log || !dt_bias || !final_state)) return GDN_ERR_NULL;
  if (T > 0 && (!q || !k || !v || !a || !b || !out)) return GDN_ERR_NULL;
  return GDN_OK;
}


// The chain kernel over the chains' grid, plus the seams' workgroups and the
// seam pass when `seams` holds any (never with h).
template <bool kL2, bool kH>
int launch_prefill(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* state,
                   const float* A_log, const uint16_t* a, const float* dt_bias, const uint16_t* b,
                   const void* cu_seqlens, int cu_is_int32, int N, int T, int HQ, int HV,
                   float scale, uint16_t* out, float* final_state, uint16_t* h, int h_chunks,
                   FusedSeams seams, int seam_ox_rows, int seam_max_tail, hipStream_t st) {
  const unsigned units = unsigned(N) * unsigned(HQ);
  const unsigned G = unsigned(HV / HQ);
  const unsigned base = 8u * G * ((units + 7u) / 8u);
  if (kH) seams.count = 0;
  seams.base_ids = int(base);
  const unsigned seam_units = unsigned(seams.count) * unsigned(HQ);
  const unsigned extra = seams.count > 0 ? 8u * 2u * G * ((seam_units + 7u) / 8u) : 0u;
  const dim3 grid{base + extra, 1u, 1u};
  const dim3 block(kThreads);
  if (cu_is_int32) {
    hipLaunchKernelGGL((gdn_prefill_chain_kernel<int32_t, kL2, kH>), grid, block, 0, st, q, k, v,
                       state, A_log, a, dt_bias, b, static_cast<const int32_t*>(cu_seqlens), N, T,
                       HQ, HV, scale, out, final_state, h, h_chunks, seams);
  } else {
    hipLaunchKernelGGL((gdn_prefill_chain_kernel<int64_t, kL2, kH>), grid, block, 0, st, q, k, v,
                       state, A_log, a, dt_bias, b, static_cast<const int64_t*>(cu_seqlens), N, T,
                       HQ, HV, scale, out, final_state, h, h_chunks, seams);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return -int(err);
  return gdn::prefill_seam_pass(seams.region, HV, seams.count, seam_ox_rows, seams.count, seam_max_tail,
                                out, final_state, st);
}

int prefill_dispatch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* state,
                     const float* A_log, const uint16_t* a, const float* dt_bias, const uint16_t* b,
                     const void* cu_seqlens, int cu_is_int32, int N, int T, int HQ, int HV,
                     float scale, uint16_t* out, float* final_state, uint16_t* h, int h_chunks,
                     int flags, hipStream_t st, const FusedSeams& seams = FusedSeams{},
                     int seam_ox_rows = 0, int seam_max_tail = 0) {
  const bool l2 = (flags & GDN_QK_L2NORM) != 0;
  if (h != nullptr) {
    return l2 ? launch_prefill<true, true>(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
                                           cu_is_int32, N, T, HQ, HV, scale, out, final_state, h,
                                           h_chunks, FusedSeams{}, 0, 0, st)
              : launch_prefill<false, true>(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
                                            cu_is_int32, N, T, HQ, HV, scale, out, final_state, h,
                                            h_chunks, FusedSeams{}, 0, 0, st);
  }
  return l2 ? launch_prefill<true, false>(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
                                          cu_is_int32, N, T, HQ, HV, scale, out, final_state,
                                          nullptr, 0, seams, seam_ox_rows, seam_max_tail, st)
            : launch_prefill<false, false>(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
                                           cu_is_int32, N, T, HQ, HV, scale, out, final_state,
                                           nullptr, 0, seams, seam_ox_rows, seam_max_tail, st);
}

}  // namespace

extern "C" size_t gdn_prefill_workspace_bytes(int N, int T, int HQ, int HV) {
  if (N <= 0 || T <= 0 || HQ <= 0 || HV <= 0 || HV % HQ != 0) return 0;
  return gdn::prefill_split_auto_slices(N, HV) > 0 ? gdn::prefill_split_workspace_bytes(N, T, HQ, HV) : 0;
}

extern "C" int gdn_prefill_auto_slices(int N, int HV) {
  if (N <= 0 || HV <= 0) return 0;
  return gdn::prefill_split_auto_slices(N, HV);
}

extern "C" size_t gdn_prefill_split_workspace_bytes(int N, int T, int HQ, int HV) {
  if (N <= 0 || T < 0 || HQ <= 0 || HV <= 0 || HV % HQ != 0) return 0;
  return gdn::prefill_split_workspace_bytes(N, T, HQ, HV);
}

extern "C" int gdn_prefill_ex_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                  const float* state, const float* A_log, const uint16_t* a,
                                  const float* dt_bias, const uint16_t* b, const void* cu_seqlens,
                                  int cu_is_int32, int N, int T, int HQ, int HV, float scale,
                                  uint16_t* out, float* final_state, void* workspace,
                                  size_t workspace_bytes, int flags, void* stream) {
  const int rc = check_prefill_args(q, k, v, A_log, a, dt_bias, b, cu_seqlens, out, final_state,
                                    N, T, HQ, HV);
  if (rc != GDN_OK) return rc;
  if (flags & ~GDN_FLAGS_ALL) return GDN_ERR_SHAPE;
  if (N == 0) return GDN_OK;
  // Few chains: split each over workgroups when the caller supplied the workspace for it.
  const int slices = T > 0 ? gdn::prefill_split_auto_slices(N, HV) : 0;
  if (slices > 0 && workspace != nullptr &&
      workspace_bytes >= gdn::prefill_split_workspace_bytes(N, T, HQ, HV)) {
    return gdn::prefill_split_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32,
                                     N, T, HQ, HV, scale, out, final_state, slices, workspace, flags,
                                     static_cast<hipStream_t>(stream));
  }
  return prefill_dispatch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N, T, HQ,
                          HV, scale, out, final_state, nullptr, 0, flags,
                          static_cast<hipStream_t>(stream));
}

extern "C" int gdn_prefill_split_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                     const float* state, const float* A_log, const uint16_t* a,
                                     const float* dt_bias, const uint16_t* b, const void* cu_seqlens,
                                     int cu_is_int32, int N, int T, int HQ, int HV, float scale,
                                     uint16_t* out, float* final_state, int slices, void* workspace,
                                     size_t workspace_bytes, int flags, void* stream) {
  const int rc = check_prefill_args(q, k, v, A_log, a, dt_bias, b, cu_seqlens, out, final_state,
                                    N, T, HQ, HV);
  if (rc != GDN_OK) return rc;
  if ((flags & ~GDN_FLAGS_ALL) || !gdn::prefill_split_slices_valid(slices)) return GDN_ERR_SHAPE;
  if (N == 0) return GDN_OK;
  const size_t need = gdn::prefill_split_workspace_bytes(N, T, HQ, HV);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return GDN_ERR_WORKSPACE;
  return gdn::prefill_split_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N,
                                   T, HQ, HV, scale, out, final_state, slices, workspace, flags,
                                   static_cast<hipStream_t>(stream));
}

extern "C" size_t gdn_prefill_split_noalloc_max_bytes(void) { return gdn::prefill_scratch_bytes(); }

extern "C" int gdn_prefill_split_noalloc_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                             const float* state, const float* A_log, const uint16_t* a,
                                             const float* dt_bias, const uint16_t* b,
                                             const void* cu_seqlens, int cu_is_int32, int N, int T,
                                             int HQ, int HV, float scale, uint16_t* out,
                                             float* final_state, int slices, int flags, void* stream) {
  const int rc = check_prefill_args(q, k, v, A_log, a, dt_bias, b, cu_seqlens, out, final_state,
                                    N, T, HQ, HV);
  if (rc != GDN_OK) return rc;
  if ((flags & ~GDN_FLAGS_ALL) || !gdn::prefill_split_slices_valid(slices)) return GDN_ERR_SHAPE;
  if (gdn::prefill_split_workspace_bytes(N, T, HQ, HV) > gdn::prefill_scratch_bytes())
    return GDN_ERR_WORKSPACE;
  if (N == 0) return GDN_OK;
  hipError_t err = hipSuccess;
  void* ws = gdn::prefill_scratch(&err);
  if (ws == nullptr) return -int(err);
  return gdn::prefill_split_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N,
                                   T, HQ, HV, scale, out, final_state, slices, ws, flags,
                                   static_cast<hipStream_t>(stream));
}

namespace {

// Cost model of the path choice, in cycles of the fused kernel's clock
// (about 2.6 GHz with at most a quarter of the CUs busy), fitted to MI355X
// timings of qk16/v32 and qk4/v8 batches (40 batches of 1-8 sequences, every
// path timed in rotation; the model's median error 5%): per chunk of a chain,
// the fused kernel 7 600 and the slice kernel 2 330 with 16 state rows
// (8 slices), 2 690 with 32 (4 slices); the split path's preparation launch
// 49 cycles per (chunk, v-head) on 256 CUs (scaled by 256 / CUs); start-up
// 24 000 cycles for the fused launch, 27 700 for the split path's two.
constexpr double kFusedChunkCycles = 7600.0;
constexpr double kSlice8ChunkCycles = 2330.0;
constexpr double kSlice4ChunkCycles = 2690.0;
constexpr double kPrepUnitCycles256 = 49.0 * 256.0;
constexpr double kStartupCycles = 24000.0;
constexpr double kSplitStartupCycles = 27700.0;
constexpr int kFusedSeamMinChunks = 8;    // shortest chain a fused seam cuts

// Finish time of workgroups that each hold one CU for `chunks * period`
// cycles, started in the given order as CUs free up, `per_seq` workgroups
// per sequence.  The workgroups of one sequence last equally long, so the
// CUs are tracked as groups that free at the same time (sorted by time).
double makespan(const std::vector<int>& chunks, int per_seq, double period, int cus) {
  std::vector<std::pair<double, long long>> free_at{{0.0, (long long)cus}};
  double end = 0.0;
  for (int n : chunks) {
    const double d = n * period;
    long long need = per_seq;
    while (need > 0 && !free_at.empty()) {
      const double t = free_at.front().first + d;
      const long long c = std::min(free_at.front().second, need);
      free_at.front().second -= c;
      if (free_at.front().second == 0) free_at.erase(free_at.begin());
      need -= c;
      end = std::max(end, t);
      auto it = std::lower_bound(free_at.begin(), free_at.end(), std::make_pair(t, 0LL));
      if (it != free_at.end() && it->first == t) it->second += c;
      else free_at.insert(it, {t, c});
    }
  }
  return end;
}

// The fused launch's seams for these lengths.  Seams take only the CUs idle
// at launch (chains < CUs): each seam's 2 HV tail workgroups start at once,
// beside the chains.  Cutting the k longest sequences (L: chunk counts,
// longest first) at chunk M, the launch ends at
//   max(M, L[k], L[0] - M + kSeamWgStartupPeriods)
// chunk periods (a workgroup's start-up, about 12 us, counts for the tails
// that start late in the serial case it replaces too little to matter), and
// the seam pass costs kSeamPassFixedCycles plus kSeamPassTokenCycles per
// (tail token, v-head) (OX rows written and read, the outputs read and
// written again).  The plan takes the k and M of the earliest modelled end,
// none when that is not earlier than the longest chain's.  `periods` is the
// modelled finish in chunk periods, the seam pass excluded.
constexpr double kSeamWgStartupPeriods = 3.5;
constexpr double kSeamPassFixedCycles = 12000.0;
constexpr double kSeamPassTokenCycles = 0.7;

struct FusedPlan {
  int count = 0;
  int seq[kMaxSeams] = {}, sp[kMaxSeams] = {}, bos[kMaxSeams] = {}, len[kMaxSeams] = {};
  int ox_row[kMaxSeams] = {};
  int ox_rows = 0, max_tail = 0, periods = 0;
};

template <typename CuT>
FusedPlan plan_fused_seams(const CuT* cu, int N, int T, int HV, int cus, bool allow) {
  FusedPlan p;
  std::vector<int> order(N), L(N), lens(N);
  for (int m = 0; m < N; ++m) {
    int bm, lm;
    seq_bounds(cu, m, T, bm, lm);
    lens[m] = lm;
    L[m] = (lm + C - 1) / C;
    order[m] = m;
  }
  const long long chains = (long long)N * HV;
  if (!allow || N == 0 || cus <= 0 || chains >= cus) {
    p.periods = N > 0 ? *std::max_element(L.begin(), L.end()) : 0;
    return p;
  }
  std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return L[x] > L[y]; });
  p.periods = L[order[0]];
  const int room = int(std::min<long long>({(cus - chains) / (2LL * HV), (long long)N, (long long)kMaxSeams}));
  const int L0 = L[order[0]];
  double best = double(L0) * kFusedChunkCycles;
  int best_k = 0, best_M = 0, best_end = L0;
  for (int k = 1; k <= room; ++k) {
    const int Lk = k < N ? L[order[k]] : 0;
    if (L[order[k - 1]] < kFusedSeamMinChunks) break;
    for (int M = std::max(1, Lk); M < L[order[k - 1]]; ++M) {
      long long tail_tokens = 0;
      for (int j = 0; j < k; ++j) tail_tokens += lens[order[j]] - (long long)C * M;
      const double end = std::max<double>({double(M), double(Lk), L0 - M + kSeamWgStartupPeriods});
      const double cost = end * kFusedChunkCycles + kSeamPassFixedCycles +
                          kSeamPassTokenCycles * double(tail_tokens) * HV;
      if (cost < best) {
        best = cost;
        best_k = k;
        best_M = M;
        best_end = int(std::ceil(end));
      }
    }
  }
  if (best_k == 0) return p;
  p.count = best_k;
  p.periods = best_end;
  for (int j = 0; j < best_k; ++j) {
    const int n = order[j];
    int bm, lm;
    seq_bounds(cu, n, T, bm, lm);
    p.seq[j] = n;
    p.sp[j] = best_M;
    p.bos[j] = bm;
    p.len[j] = lm;
    p.ox_row[j] = p.ox_rows;
    p.ox_rows += lm - C * best_M;
    p.max_tail = std::max(p.max_tail, L[n] - best_M);
  }
  return p;
}

// Slices of the split path (4 / 8) or 0 for the fused kernel, from the modelled
// times of the three for these lengths; the fused kernel's with the seams of
// fp, the split path's with the seams its launch chooses on the device
// (HQ > 0; HQ = 0: none).
template <typename CuT>
int choose_path(const CuT* cu, int N, int T, int HQ, int HV, int cus, const FusedPlan& fp) {
  const long long chains = (long long)N * HV;
  // Past one chain per CU the fused kernel fills the GPU and the split path
  // would need 4 or 8 times as many workgroups.
  if (N == 0 || cus <= 0 || chains > cus) return 0;
  std::vector<int> chunks(N);
  double units = 0.0;
  for (int m = 0; m < N; ++m) {
    int bm, lm;
    seq_bounds(cu, m, T, bm, lm);
    chunks[m] = (lm + C - 1) / C;
    units += double(chunks[m]) * HV;
  }
  // one fused workgroup per chain, all resident at once (chains <= CUs)
  long long tail_tokens = 0;
  for (int j = 0; j < fp.count; ++j) tail_tokens += fp.len[j] - (long long)C * fp.sp[j];
  const double fused = kStartupCycles + fp.periods * kFusedChunkCycles +
                       (fp.count ? kSeamPassFixedCycles + kSeamPassTokenCycles * double(tail_tokens) * HV : 0.0);
  // the slice launch takes the sequences longest first
  std::sort(chunks.begin(), chunks.end(), std::greater<int>());
  const double prep = kSplitStartupCycles + units * kPrepUnitCycles256 / cus;
  auto split = [&](int slices, double period) {
    const int room = HQ > 0 ? gdn::prefill_split_seam_room(N, HQ, HV, slices, cus) : 0;
    int seams = 0;
    const int span = gdn::prefill_split_seam_span(chunks.data(), N, room, &seams);
    // with seams every workgroup is resident: the span is the finish
    return prep + (seams > 0 ? span * period : makespan(chunks, HV * slices, period, cus));
  };
  const double split8 = split(8, kSlice8ChunkCycles);
  const double split4 = split(4, kSlice4ChunkCycles);
  if (split8 <= split4 && split8 < fused) return 8;
  if (split4 < fused) return 4;
  return 0;
}

// The plan behind gdn_prefill_plan / gdn_prefill_plan_fwd (host memory, opaque
// to callers).
constexpr uint32_t kPlanMagic = 0x50444e47u;   // "GNDP", layout 1
struct PrefillPlan {
  uint32_t magic;
  int N, T, HQ, HV;
  int slices;                 // 4 / 8: the split path; 0: the fused kernel
  int split_seams;            // seam slots the split launch reserves
  FusedPlan fused;            // the fused kernel's seams
  unsigned long long workspace_bytes;
};
static_assert(sizeof(PrefillPlan) <= GDN_PREFILL_PLAN_BYTES, "plan size");

template <typename CuT>
void make_plan(const CuT* cu, int N, int T, int HQ, int HV, int cus, bool seams, bool fused_only,
               PrefillPlan& p) {
  p = PrefillPlan{};
  p.magic = kPlanMagic;
  p.N = N;
  p.T = T;
  p.HQ = HQ;
  p.HV = HV;
  p.fused = plan_fused_seams(cu, N, T, HV, cus, seams && T > 0);
  p.slices = T > 0 && !fused_only ? choose_path(cu, N, T, seams ? HQ : 0, HV, cus, p.fused) : 0;
  if (p.slices) {
    p.fused = FusedPlan{};
    p.split_seams = seams ? gdn::prefill_split_seam_room(N, HQ, HV, p.slices, cus) : 0;
    p.workspace_bytes = gdn::prefill_split_workspace_bytes(N, T, HQ, HV);
  } else {
    p.workspace_bytes = p.fused.count ? seam_region_bytes(p.fused.count, HV, p.fused.ox_rows) : 0;
  }
}

}  // namespace

extern "C" int gdn_prefill_choose_slices(const void* cu_seqlens_host, int cu_is_int32, int N, int T,
                                         int HV, int cus) {
  if (!cu_seqlens_host || N < 0 || T < 0 || HV <= 0) return -1;
  if (cus <= 0) cus = gdn::device_cus();
  if (N == 0 || cus <= 0 || (long long)N * HV > cus) return 0;
  // the fused kernel as gdn_prefill_ex_fwd runs it without a workspace: no seams
  if (cu_is_int32) {
    const auto* cu = static_cast<const int32_t*>(cu_seqlens_host);
    return choose_path(cu, N, T, 0, HV, cus, plan_fused_seams(cu, N, T, HV, cus, false));
  }
  const auto* cu = static_cast<const int64_t*>(cu_seqlens_host);
  return choose_path(cu, N, T, 0, HV, cus, plan_fused_seams(cu, N, T, HV, cus, false));
}

extern "C" int gdn_prefill_plan(const void* cu_seqlens_host, int cu_is_int32, int N, int T, int HQ,
                                int HV, int cus, int flags, void* plan, size_t* workspace_bytes) {
  if (!cu_seqlens_host || !plan) return GDN_ERR_NULL;
  if (N < 0 || T < 0 || HQ <= 0 || HV <= 0 || HV % HQ != 0 || (flags & ~(GDN_FLAGS_ALL | GDN_PLAN_FUSED)))
    return GDN_ERR_SHAPE;
  if (cus <= 0) cus = gdn::device_cus();
  PrefillPlan p;
  const bool seams = (flags & GDN_NO_SEAMS) == 0, fused = (flags & GDN_PLAN_FUSED) != 0;
  if (cu_is_int32) make_plan(static_cast<const int32_t*>(cu_seqlens_host), N, T, HQ, HV, cus, seams, fused, p);
  else make_plan(static_cast<const int64_t*>(cu_seqlens_host), N, T, HQ, HV, cus, seams, fused, p);
  std::memcpy(plan, &p, sizeof(p));
  if (workspace_bytes) *workspace_bytes = size_t(p.workspace_bytes);
  return GDN_OK;
}

extern "C" int gdn_prefill_plan_info(const void* plan, int* slices, int* seams, int* split_chunk,
                                     int* periods) {
  if (!plan) return GDN_ERR_NULL;
  PrefillPlan p;
  std::memcpy(&p, plan, sizeof(p));
  if (p.magic != kPlanMagic) return GDN_ERR_SHAPE;
  if (slices) *slices = p.slices;
  if (seams) *seams = p.slices ? p.split_seams : p.fused.count;
  if (split_chunk) *split_chunk = p.fused.count ? p.fused.sp[0] : 0;
  if (periods) *periods = p.fused.periods;
  return GDN_OK;
}

extern "C" int gdn_prefill_plan_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    const float* state, const float* A_log, const uint16_t* a,
                                    const float* dt_bias, const uint16_t* b, const void* cu_seqlens,
                                    int cu_is_int32, int N, int T, int HQ, int HV, float scale,
                                    uint16_t* out, float* final_state, const void* plan,
                                    void* workspace, size_t workspace_bytes, int flags, void* stream) {
  const int rc = check_prefill_args(q, k, v, A_log, a, dt_bias, b, cu_seqlens, out, final_state,
                                    N, T, HQ, HV);
  if (rc != GDN_OK) return rc;
  if (!plan) return GDN_ERR_NULL;
  if (flags & ~GDN_FLAGS_ALL) return GDN_ERR_SHAPE;
  PrefillPlan p;
  std::memcpy(&p, plan, sizeof(p));
  if (p.magic != kPlanMagic || p.N != N || p.T != T || p.HQ != HQ || p.HV != HV) return GDN_ERR_SHAPE;
  if (p.fused.count < 0 || p.fused.count > kMaxSeams || (p.slices && !gdn::prefill_split_slices_valid(p.slices)))
    return GDN_ERR_SHAPE;
  if (N == 0) return GDN_OK;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.slices) {
    const size_t need = gdn::prefill_split_workspace_bytes(N, T, HQ, HV);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return GDN_ERR_WORKSPACE;
    return gdn::prefill_split_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N,
                                     T, HQ, HV, scale, out, final_state, p.slices, workspace, flags, st);
  }
  FusedSeams seams{};
  if (p.fused.count > 0 && !(flags & GDN_NO_SEAMS)) {
    const size_t need = seam_region_bytes(p.fused.count, HV, p.fused.ox_rows);
    if (workspace == nullptr || workspace_bytes < need) return GDN_ERR_WORKSPACE;
    // A plan is checked against itself before it sizes any write: every
    // tail inside [0, T), the OX rows of seam j at the running sum of the
    // tails before it and the region sized for all of them, the seam pass's
    // pieces covering the longest tail, no sequence cut twice.
    const FusedPlan& f = p.fused;
    long long rows = 0;
    int max_tail = 0;
    for (int j = 0; j < f.count; ++j) {
      if (f.seq[j] < 0 || f.seq[j] >= N || f.bos[j] < 0 || f.len[j] < 0 || (long long)f.bos[j] + f.len[j] > T ||
          f.sp[j] < 1 || C * (long long)f.sp[j] >= f.len[j] || f.ox_row[j] != rows)
        return GDN_ERR_SHAPE;
      for (int i = 0; i < j; ++i)
        if (f.seq[i] == f.seq[j]) return GDN_ERR_SHAPE;
      rows += f.len[j] - (long long)C * f.sp[j];
      max_tail = std::max(max_tail, (f.len[j] + C - 1) / C - f.sp[j]);
    }
    if (rows != f.ox_rows || max_tail != f.max_tail) return GDN_ERR_SHAPE;
    seams.count = p.fused.count;
    for (int j = 0; j < seams.count; ++j) {
      seams.seq[j] = p.fused.seq[j];
      seams.sp[j] = p.fused.sp[j];
      seams.bos[j] = p.fused.bos[j];
      seams.len[j] = p.fused.len[j];
      seams.ox_row[j] = p.fused.ox_row[j];
    }
    seams.region = static_cast<char*>(workspace);
  }
  return prefill_dispatch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N, T, HQ, HV,
                          scale, out, final_state, nullptr, 0, flags, st, seams, p.fused.ox_rows,
                          p.fused.max_tail);
}

extern "C" long long gdn_prefill_chunk_count(const void* cu_seqlens_host, int cu_is_int32, int N,
                                             int T) {
  if (!cu_seqlens_host || N < 0 || T < 0) return -1;
  long long total = 0;
  for (int m = 0; m < N; ++m) {
    int bm, lm;
    if (cu_is_int32) seq_bounds(static_cast<const int32_t*>(cu_seqlens_host), m, T, bm, lm);
    else seq_bounds(static_cast<const int64_t*>(cu_seqlens_host), m, T, bm, lm);
    total += (lm + C - 1) / C;
  }
  return total;
}

extern "C" int gdn_prefill_h_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const float* state, const float* A_log, const uint16_t* a,
                                 const float* dt_bias, const uint16_t* b, const void* cu_seqlens,
                                 int cu_is_int32, int N, int T, int HQ, int HV, float scale,
                                 uint16_t* out, float* final_state, uint16_t* h, int h_chunks,
                                 void* workspace, size_t workspace_bytes, int flags, void* stream) {
  const int rc = check_prefill_args(q, k, v, A_log, a, dt_bias, b, cu_seqlens, out, final_state,
                                    N, T, HQ, HV);
  if (rc != GDN_OK) return rc;
  if (!h && h_chunks > 0) return GDN_ERR_NULL;
  if (h_chunks < 0 || (flags & ~GDN_FLAGS_ALL)) return GDN_ERR_SHAPE;
  if (N == 0) return GDN_OK;
  // Few chains: the split path when the caller supplied its workspace, as gdn_prefill_ex_fwd.
  const int slices = T > 0 ? gdn::prefill_split_auto_slices(N, HV) : 0;
  if (slices > 0 && workspace != nullptr &&
      workspace_bytes >= gdn::prefill_split_workspace_bytes(N, T, HQ, HV)) {
    return gdn::prefill_split_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32,
                                     N, T, HQ, HV, scale, out, final_state, slices, workspace, flags,
                                     static_cast<hipStream_t>(stream), h, h_chunks);
  }
  return prefill_dispatch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N, T, HQ,
                          HV, scale, out, final_state, h, h_chunks, flags,
                          static_cast<hipStream_t>(stream));
}

extern "C" int gdn_prefill_split_h_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                       const float* state, const float* A_log, const uint16_t* a,
                                       const float* dt_bias, const uint16_t* b,
                                       const void* cu_seqlens, int cu_is_int32, int N, int T, int HQ,
                                       int HV, float scale, uint16_t* out, float* final_state,
                                       uint16_t* h, int h_chunks, int slices, void* workspace,
                                       size_t workspace_bytes, int flags, void* stream) {
  const int rc = check_prefill_args(q, k, v, A_log, a, dt_bias, b, cu_seqlens, out, final_state,
                                    N, T, HQ, HV);
  if (rc != GDN_OK) return rc;
  if (!h && h_chunks > 0) return GDN_ERR_NULL;
  if (h_chunks < 0 || (flags & ~GDN_FLAGS_ALL) || !gdn::prefill_split_slices_valid(slices))
    return GDN_ERR_SHAPE;
  if (N == 0) return GDN_OK;
  const size_t need = gdn::prefill_split_workspace_bytes(N, T, HQ, HV);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return GDN_ERR_WORKSPACE;
  return gdn::prefill_split_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N,
                                   T, HQ, HV, scale, out, final_state, slices, workspace, flags,
                                   static_cast<hipStream_t>(stream), h, h_chunks);
}

extern "C" int gdn_prefill_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const float* state, const float* A_log, const uint16_t* a,
                               const float* dt_bias, const uint16_t* b, const void* cu_seqlens,
                               int cu_is_int32, int N, int T, int HQ, int HV, float scale,
                               uint16_t* out, float* final_state, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return gdn_prefill_ex_fwd(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_is_int32, N, T, HQ,
                            HV, scale, out, final_state, workspace, workspace_bytes, 0, stream);
}
