// Device helpers shared by the GDN prefill kernels (gfx950 / CDNA4, wave64):
// chunk geometry, LDS operand layouts, MFMA wrappers, HBM->LDS copies and
// barriers.  Used by the fused chain kernel (gdn_prefill.hip) and by the
// chunk-preparation and state-slice kernels (gdn_prefill_split.hip).
#pragma once

#include <type_traits>

#include "gdn_common.h"

namespace gdn {

constexpr int D = kHeadDim;   // 128
constexpr int C = 64;         // chunk
// Row strides, chosen so that the MFMA operand reads (16-byte reads down 16
// rows, and the transposing 8-byte reads down 4 rows x 4 quads) are free of
// LDS bank conflicts: rows of 288 B (Kc, A) and 160 B (Tm / P).
constexpr int KCLD = D + 16;  // Kc row stride (halves): 288 B rows
constexpr int TLD = C + 16;   // Tm / P row stride (halves): 160 B rows
constexpr int ALD = C + 8;    // A row stride (floats): 288 B rows
constexpr int BLD = C / 2 + 8;  // Aba row stride (halves): 80 B rows
// Gate data per chunk, GSZ floats: gam log2(e) | beta | e^gam | scale e^gam | e^(gam_L - gam)
// (gam = chunk-local cumsum of the log-decay, gam_L its value at the chunk's last token).
constexpr int G_L2 = 0, G_BETA = C, G_EG = 2 * C, G_EGS = 3 * C, G_ED = 4 * C;
constexpr int GSZ = 5 * C;

typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// Column order inside every 32-column group of the fp16 operand tiles: column
// 16 a + 4 q + r is stored at position 8 q + 4 a + r.  The 8 k-slots that
// lane group q feeds a 16x16x32 MFMA from two stacked 16x16 accumulator tiles
// -- rows 4q..4q+3 of each -- are then 16 contiguous bytes, and every quad
// of 4 consecutive columns stays contiguous.
__device__ __forceinline__ int p32(int c) {
  return (c & ~31) | (((c >> 2) & 3) << 3) | (((c >> 4) & 1) << 2) | (c & 3);
}

// Raw bf16 rows as copied from HBM: 16-byte chunk c of row t sits in slot
// c ^ (t & 15) of that row (the copy picks which global chunk each lane
// fetches), so column reads down 16 consecutive rows hit 16 distinct banks.
__device__ __forceinline__ int raw_off(int t, int col) { return t * D + 8 * ((col >> 3) ^ (t & 15)) + (col & 7); }

struct __align__(16) SmemRaw {
  uint16_t k[2][C * D];        // K rows of the chunks of parity 0 / 1 (bf16, swizzled), DMA target
  uint16_t q[2][C * D];        // Q rows of the chunks of parity 0 / 1 (bf16, swizzled), DMA target
};

struct __align__(16) Smem {
  _Float16 Kc[2][C * KCLD];    // K chunk in fp16 [t][p32(k)], double-buffered
  _Float16 Tm[C * TLD];        // diagonal 32-row blocks of (I + A)^-1 [t][p32(t')]
  _Float16 P[C * TLD];         // decayed causal Q K^T [t][p32(t')]
  float A[C * ALD];            // beta-scaled decayed strict K K^T [t][t'] (fp32), diagonal 32-row blocks
  _Float16 Aba[(C / 2) * BLD]; // its lower-left 32x32 block, negated, in fp16 [t - 32][p32(t')]
};

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for outstanding global stores or HBM->LDS copies.  The asm
// statement is a compiler memory barrier as well.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Workgroup barrier that leaves up to N of this wave's most recent LDS reads
// in flight.  For a wave that reads LDS and never writes it: every read whose
// value it has used before the barrier has completed, and what may still be
// outstanding are reads whose values are used after it -- reads of data that
// no wave overwrites in the next phase.
template <int N>
__device__ __forceinline__ void lds_barrier_keep() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)\n\ts_barrier" :: "n"(N) : "memory");
}

// Waits until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

__device__ __forceinline__ f16x8 ld16(const _Float16* p) { return *reinterpret_cast<const f16x8*>(p); }

__device__ __forceinline__ bf16x8_t ld16_bf(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}

// Transposing LDS read (ds_read_b64_tr_b16): inside each 16-lane group, lane i
// receives element i % 4 of the 8-byte reads issued by lanes 4 m + i / 4,
// m = 0..3, of the same group.
__device__ __forceinline__ f16x4_t ld_tr16(const _Float16* p) {
  return __builtin_bit_cast(f16x4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                         (__attribute__((address_space(3))) i16x4_t*)p));
}

__device__ __forceinline__ f16x8 ld_f32x8_as_f16(const float* p) {
  const f32x4 lo = *reinterpret_cast<const f32x4*>(p);
  const f32x4 hi = *reinterpret_cast<const f32x4*>(p + 4);
  return f16x8{(_Float16)lo[0], (_Float16)lo[1], (_Float16)lo[2], (_Float16)lo[3],
               (_Float16)hi[0], (_Float16)hi[1], (_Float16)hi[2], (_Float16)hi[3]};
}

// Two stacked 16x16 accumulator tiles -> one 8-slot fp16 operand.
__device__ __forceinline__ f16x8 pack2(const f32x4& a, const f32x4& b) {
  return f16x8{(_Float16)a[0], (_Float16)a[1], (_Float16)a[2], (_Float16)a[3],
               (_Float16)b[0], (_Float16)b[1], (_Float16)b[2], (_Float16)b[3]};
}

// Two stacked 16x16 accumulator tiles -> one 8-slot bf16 operand.
__device__ __forceinline__ bf16x8_t pack2_bf(const f32x4& a, const f32x4& b) {
  return bf16x8_t{(__bf16)a[0], (__bf16)a[1], (__bf16)a[2], (__bf16)a[3],
                  (__bf16)b[0], (__bf16)b[1], (__bf16)b[2], (__bf16)b[3]};
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

__device__ __forceinline__ f32x4 mfma16_bf(bf16x8_t a, bf16x8_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16k16(f16x4_t a, f16x4_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Row of accumulator element i for lane half h (32x32 layout).
__device__ __forceinline__ int acc_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// HBM -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane l's
// bytes land at lds_dst + 16 l; lds_dst must be uniform across the wave.
// Issued from asm so that the compiler does not wait for it at LDS accesses
// it cannot tell apart from the destination; every consumer of the copied
// data waits for it explicitly (wait_vm) and then crosses a barrier.  The
// LDS address goes in through a fixed M0 operand ("{m0}"): the compiler
// writes M0 itself and knows what it holds; the s_nop separates that write
// from the load that reads it.
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_dst) {
  const uint32_t lds_addr = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds_dst);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(src), "{m0}"(lds_addr) : "memory");
}

// The same copy from base + off: base uniform (an SGPR pair), off a 32-bit
// lane offset (no 64-bit address arithmetic per copy).
__device__ __forceinline__ void lds_dma16_saddr(const void* base, uint32_t off, void* lds_dst) {
  const uint32_t lds_addr = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds_dst);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(off), "s"(base), "{m0}"(lds_addr) : "memory");
}

// Round-to-nearest-even fp32 pair -> packed bf16 pair (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16 bytes to base + off: base uniform (an SGPR pair), off a 32-bit lane offset.
// Nothing in the kernel reads what these stores write.
// A store of more than 8 bytes keeps reading its data VGPRs after issue: a
// VALU write to them needs 2 wait states first (the compiler counts them for
// its own stores, not for this asm), hence the s_nop.
__device__ __forceinline__ void store_b128_saddr(char* base, uint32_t off, u32x4_t data) {
  asm volatile("global_store_dwordx4 %0, %1, %2\n\ts_nop 1" :: "v"(off), "v"(data), "s"(base)
               : "memory");
}

// Raw buffer resource (stride 0) over `bytes` bytes from `base`, both made
// wave-uniform.  A buffer access whose offset is at or past `bytes` is out of
// range: a store there writes nothing.  Such stores mask rows without a
// branch, so every path through a loop issues the same memory instructions
// and the compiler's vmcnt waits for earlier loads stay exact.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_buffer(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  void* p = reinterpret_cast<void*>((uint64_t(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, short(0), int(__builtin_amdgcn_readfirstlane(bytes)), 0x00020000);
}

// Offset that lands out of range of every buffer uniform_buffer makes.
constexpr uint32_t kBufferDrop = 0x80000000u;

__device__ __forceinline__ void buffer_store_b64(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t lo,
                                                 uint32_t hi) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{lo, hi}, r, int(off), 0, 0);
}

// The bf16 image of a 16-row tile of the state to a row-major [16][128]
// bf16 destination (an h slot), column blocks 2 pp and 2 pp + 1 (s0, s1)
// at a time, as whole 128-byte lines.  Lane (g, c) holds row c of the tile,
// 4-column pieces g and g + 4 of each block (the S^T accumulator layout
// packed to bf16).  v_permlane16_swap trades the odd 16-lane rows' first
// piece for the even rows' second, which leaves every lane two adjacent
// pieces of each block (16 contiguous bytes: x of block 2 pp, y of block
// 2 pp + 1): pieces g, g + 1 (g even) or g + 3, g + 4 (g odd).  A DPP
// rotation by 8 within each 16-lane row gives lane c the x and y of lane
// c ^ 8, so the first store writes rows c % 8 (x on lanes c < 8, the y of
// row c - 8 on the others) and the second rows c % 8 + 8: 8 whole lines
// each, where one store per block would write 16 half lines.  (Used by the
// fused chain kernel, where all 256 CUs write h at once.)
// `tile` points at the tile's row 0, column 64 pp; lane_off is
// state_lines_lane(g, c).
__device__ __forceinline__ uint32_t state_lines_lane(int g, int c) {
  return uint32_t((c & 7) * 128 + ((g & 1) ? 4 * (g + 3) : 4 * g)) * 2u + ((c & 8) ? 64u : 0u);
}
__device__ __forceinline__ void store_state_lines(char* tile, uint32_t lane_off, int c, bf16x8_t s0,
                                                  bf16x8_t s1) {
  const u32x4_t w0 = __builtin_bit_cast(u32x4_t, s0);
  const u32x4_t w1 = __builtin_bit_cast(u32x4_t, s1);
  const auto a0 = __builtin_amdgcn_permlane16_swap(w0[0], w0[2], false, false);
  const auto a1 = __builtin_amdgcn_permlane16_swap(w0[1], w0[3], false, false);
  const auto b0 = __builtin_amdgcn_permlane16_swap(w1[0], w1[2], false, false);
  const auto b1 = __builtin_amdgcn_permlane16_swap(w1[1], w1[3], false, false);
  const uint32_t x[4] = {a0[0], a1[0], a0[1], a1[1]};
  const uint32_t y[4] = {b0[0], b1[0], b0[1], b1[1]};
  const bool low = (c & 8) == 0;
  u32x4_t d1, d2;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t rx = __builtin_amdgcn_update_dpp(0u, x[e], 0x128, 0xf, 0xf, false);   // row_ror:8
    const uint32_t ry = __builtin_amdgcn_update_dpp(0u, y[e], 0x128, 0xf, 0xf, false);
    d1[e] = low ? x[e] : ry;
    d2[e] = low ? rx : y[e];
  }
  store_b128_saddr(tile, lane_off, d1);
  store_b128_saddr(tile, lane_off + 8u * 128u * 2u, d2);
}

// Tokens [bos, bos + len) of sequence n, clamped into [0, T].
template <typename CuT>
__host__ __device__ __forceinline__ void seq_bounds(const CuT* cu, int n, int T, int& bos, int& len) {
  long long b0 = (long long)cu[n], e0 = (long long)cu[n + 1];
  b0 = b0 < 0 ? 0 : (b0 > T ? T : b0);
  e0 = e0 < b0 ? b0 : (e0 > T ? T : e0);
  bos = int(b0);
  len = int(e0 - b0);
}

// ---------------------------------------------------------------------------
// Seams: time splits of long chains, on either prefill path.  Sequence n of
// Lc chunks cut at chunk sp runs its head [0, sp) from the initial state and,
// at the same time, its tail [sp, Lc) twice: from a zero state (outputs O0,
// final state S0) and as the transition chain (v = 0, initial state the
// identity; its state X is the product of the tail's per-chunk transitions,
// its outputs OX the outputs' part linear in the state entering the tail).
// With S_sp the head's final state the tail outputs are O0 + OX S_sp^T and
// the final state S_sp X + S0, which the seam pass forms.
//
// A seam region of the workspace holds the plan (kSeamPlanStride ints per
// seam slot, fields SeamPlanField, sequence -1 in unused slots), then per
// slot and v-head three fp32 [128][128] states (the head's final state, the
// tail's zero-state final state, X stored transposed), then the OX rows of
// the seams' tail tokens, bf16 [ox_rows][HV][128], seam j from row
// SP_OX_ROW on.
constexpr int kMaxSeams = 8;
constexpr int kSeamPlanStride = 8;
enum SeamPlanField { SP_SEQ, SP_BOS, SP_LEN, SP_SPLIT, SP_CHUNKS, SP_OX_ROW };
constexpr size_t kSeamPlanBytes = 512;
static_assert(size_t(kSeamPlanStride) * kMaxSeams * sizeof(int) <= kSeamPlanBytes, "seam plan");
constexpr size_t kSeamStateBytes = size_t(D) * D * 4;
// kind: 0 the head's final state, 1 the tail's zero-state final state, 2 X^T
__host__ __device__ inline size_t seam_state_offset(int HV, int j, int hv, int kind) {
  return kSeamPlanBytes + ((size_t(j) * HV + hv) * 3 + kind) * kSeamStateBytes;
}
__host__ __device__ inline size_t seam_ox_offset(int k_slots, int HV) {
  return kSeamPlanBytes + size_t(k_slots) * HV * 3 * kSeamStateBytes;
}
__host__ __device__ inline size_t seam_region_bytes(int k_slots, int HV, int ox_rows) {
  return seam_ox_offset(k_slots, HV) + size_t(ox_rows) * HV * D * 2;
}

// Lower 16x16 tiles of a 64x64 chunk matrix, row-major: tile -> (ti, tj).
template <int TILE>
struct Tile16 {
  static constexpr int ti = TILE < 1 ? 0 : TILE < 3 ? 1 : TILE < 6 ? 2 : 3;
  static constexpr int tj = TILE - (ti * (ti + 1)) / 2;
};
template <int N>
using IC = std::integral_constant<int, N>;


// Inclusive prefix sum of an int over the 64 lanes of a wave.
__device__ __forceinline__ int wave_scan_incl(int x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  return x;
}

// Sequence n and chunk i of chunk slot `slot` = chunk_offset(n) + i, where
// chunk_offset(n) counts the 64-token chunks of sequences 0 .. n-1 (lengths
// clamped as seq_bounds clamps them).  n = -1 past the last chunk.
// Wave-uniform result.  The reference builds the same (sequence, chunk)
// table on the host (prepare_chunk_indices, kernel.py:175-202).
template <typename CuT>
__device__ void locate_chunk(const CuT* cu, int N, int T, int slot, int lane, int& n, int& ci) {
  int base = 0;
  n = -1;
  ci = 0;
  for (int m0 = 0; m0 < N; m0 += 64) {
    const int m = m0 + lane;
    int cnt = 0;
    if (m < N) {
      int bm, lm;
      seq_bounds(cu, m, T, bm, lm);
      cnt = (lm + C - 1) / C;
    }
    const int incl = wave_scan_incl(cnt, lane);
    const unsigned long long hit = __ballot(base + incl > slot);
    if (hit) {
      const int first = __ffsll((long long)hit) - 1;
      n = m0 + first;
      ci = slot - base - __shfl(incl - cnt, first);
      return;
    }
    base += __shfl(incl, 63);
  }
}

// chunk_offset(n) (wave-uniform): lanes take every 64th sequence, then a wave sum.
template <typename CuT>
__device__ int chunk_offset(const CuT* cu, int n, int T, int lane) {
  int part = 0;
  for (int m = lane; m < n; m += 64) {
    int bm, lm;
    seq_bounds(cu, m, T, bm, lm);
    part += (lm + C - 1) / C;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  return __builtin_amdgcn_readfirstlane(part);
}

}  // namespace gdn
