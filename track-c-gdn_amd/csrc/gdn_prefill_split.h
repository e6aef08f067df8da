// Host-side interface of the split prefill path (gdn_prefill_split.hip): a
// parallel chunk-preparation launch followed by a launch of state slices,
// for batches with fewer (sequence, v-head) chains than the GPU has CUs.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gdn {

// Workspace bytes of the split path for an upper bound of T / 64 + N chunks:
// one 14 080-byte record per (chunk, v-head) and one 18 432-byte fp16 K image
// per (chunk, qk-head), then the sequences' launch order (N ints, rounded up
// to 256 bytes).
size_t prefill_split_workspace_bytes(int N, int T, int HQ, int HV);

// Slices per chain the split path uses on the current device for N * HV
// chains: 8 when chains * 8 fit the CUs, 4 when chains * 4 fit twice the
// CUs, else 0 (the fused chain kernel runs).
int prefill_split_auto_slices(int N, int HV);

bool prefill_split_slices_valid(int slices);

// CUs of the current device (looked up once per device), 0 on error.
int device_cus();

// Size and current-device address of the library's static split-path
// workspace (the allocation-free entry point's scratch).
size_t prefill_scratch_bytes();
void* prefill_scratch(hipError_t* err);

// Enqueues both launches on st; workspace holds prefill_split_workspace_bytes.
// With h non-NULL the slices also write the bf16 state entering every chunk
// to h[chunk_offset(n) + i] for slots below h_chunks.
// Seam slots the split launch reserves for N sequences of HQ qk-heads and HV
// v-heads in `slices` slices on `cus` CUs (the seams themselves are chosen on
// the device; 0: no seam pass).
int prefill_split_seam_room(int N, int HQ, int HV, int slices, int cus);

// The seams the split launch chooses within `room` slots for sequences of
// these chunk counts (longest first, N of them): their count in *seams (may
// be NULL) and the modelled finish in chunk periods of a slice (the seam
// pass included; the longest chain's chunks without seams).
int prefill_split_seam_span(const int* chunks_desc, int N, int room, int* seams);

// Seam pass over a seam region (layout in gdn_prefill_common.h) of k_slots
// slots and ox_rows OX rows: for the first `seams` slots, the final states
// and the tail outputs' correction, max_tail_chunks bounding every seam's
// tail chunks.  Enqueued on st.
int prefill_seam_pass(char* region, int HV, int k_slots, int ox_rows, int seams, int max_tail_chunks,
                      uint16_t* out, float* final_state, hipStream_t st);

int prefill_split_launch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* state,
                         const float* A_log, const uint16_t* a, const float* dt_bias,
                         const uint16_t* b, const void* cu_seqlens, int cu_is_int32, int N, int T,
                         int HQ, int HV, float scale, uint16_t* out, float* final_state,
                         int slices, void* workspace, int flags, hipStream_t st,
                         uint16_t* h = nullptr, int h_chunks = 0);

}  // namespace gdn
