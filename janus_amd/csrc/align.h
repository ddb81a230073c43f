// Internal interface of the align kernels (align.hip), shared with the pipelines that build a GEMM chunk list.
#pragma once

#include "common.h"

namespace janus {

constexpr int kMaxExperts = 1024;  // one scan thread per expert
constexpr int kAlignChunk = 1024;  // assignments per rank/scatter block

struct AlignWorkspace {
  int* hist;        // [nb][E] per-block counts, then per-block offsets
  int* local_rank;  // [A]
  int* counts;      // [E]
  int* start;       // [E] padded start of each expert's rows
};

AlignWorkspace carve_align(Carver& c, int A, int E);

// sorted_ids [sorted_len] gets the permutation, the sentinel A everywhere else. Either expert_ids/total (reference tile
// plan, `tiles` entries) or chunks/num_chunks (runs of at most chunk_rows rows of one expert) may be null. clear[0 ..
// clear_n) is set to zero on the side (the counters of a later launch; null when clear_n == 0). Ids outside [0, E)
// are dropped; status (null: no report) gets kStatusDroppedIds when one is.
template <typename IdxT, typename OutT>
int launch_align(const IdxT* idx, int A, int E, int block, const AlignWorkspace& w, OutT* sorted_ids, int sorted_len,
                 OutT* expert_ids, int tiles, OutT* total, int4* chunks, int chunk_rows, int* num_chunks, int* clear,
                 int clear_n, int* status, hipStream_t stream);

// The GEMM chunk list and int32 permutation from a caller's reference tile plan (sorted_ids [tiles * block],
// expert_ids [tiles], int64, as align() returns them for some block), in place of an align launch; clear[0 .. clear_n)
// is zeroed as align does.
int launch_plan_chunks(const int64_t* plan_sorted_ids, const int64_t* plan_expert_ids, int tiles, int block, int A,
                       int E, int* sorted_ids, int4* chunks, int capacity, int chunk_rows, int* num_chunks, int* clear,
                       int clear_n, hipStream_t stream);

}  // namespace janus
