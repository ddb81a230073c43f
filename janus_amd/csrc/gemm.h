// Internal interface of the grouped W4A16 GEMM kernels (gemm.hip).
#pragma once

#include "common.h"

namespace janus {

constexpr int kRowBlocks = 6;                 // MFMA row blocks per workgroup tile
constexpr int kChunkRows = 16 * kRowBlocks;   // rows of one expert (or shared-expert tokens) per workgroup
constexpr int kRowPad = 16;                   // every expert's rows start at a multiple of this in the permuted order

// Rows per chunk for a call: 96 (the 6-row-block tile), or 16 (a one-row-block tile, three workgroups per CU) when the
// assignments average at most 4 rows per expert, where nearly every expert fits one 16-row chunk and the launch is
// bound by the weight decode rather than by MFMA (the shorter tile frees the accumulator registers for more waves).
inline int chunk_rows_for(long assignments, int E) { return assignments <= 4l * E ? 16 : kChunkRows; }

// Slots: each weighted expert output row (one token, one top-k slot; slot top_k is the gated shared expert) is kept
// as int16 codes with one fp32 scale per block of kSlotBlock columns, value = code * scale. The down epilogue maps
// the block's largest |value| to code 32767, so a value's error is at most scale / 2 (2^-16 of the block maximum).
// Within a block the 16 groups of 4 columns are stored in the order the epilogue's lanes hold them: true group g
// sits at stored group slot_stored_group(g).
constexpr int kSlotBlock = 64;
__host__ __device__ inline int slot_stored_group(int g) { return (g & 8) | ((g & 3) << 1) | ((g >> 2) & 1); }
// The values of one stored group: four int16 codes (two per word, low half first) times the block's scale.
__device__ __forceinline__ float4 slot_decode4(uint2 v, float scale) {
  return make_float4((float)(int16_t)(v.x & 0xFFFFu) * scale, (float)((int32_t)v.x >> 16) * scale,
                     (float)(int16_t)(v.y & 0xFFFFu) * scale, (float)((int32_t)v.y >> 16) * scale);
}

// One grouped GEMM launch over a chunk list (routed experts) plus, optionally, the shared expert as n_shared_chunks
// chunks of consecutive tokens.
//   gate_up: h[row, n] = bf16(silu(x[tok] . Wg[n]) * (x[tok] . Wu[n])) for n < I, W rows 0..I-1 gate, I..2I-1 up.
//   down:    slot (tok, slot) = w(row) * (h[row] . Wd[n]), slot = the assignment's top-k slot, or top_k for the shared
//            expert (weight sigmoid gate), encoded as above. A combine pass sums the slots of each token.
struct GemmParams {
  const uint16_t* a;          // gate_up: x [T, K]; down: h of the routed rows [P, K]
  const uint16_t* a_sh;       // down: h of the shared expert [T, K_sh]
  uint32_t a_bytes, a_sh_bytes;  // sizes of a and a_sh (below 2 GiB): loads past them read zeros
  const int* sorted_ids;      // assignment id at each permuted position (< A on real rows)
  int topk, A, T;
  int codec;                  // 0: int4 group-128 (q words, s bf16 [E, N, K/128]); 1: NVFP4 (q bytes, s e4m3
                              // [E, N, K/16], gsc fp32 [E, N]); the shared expert uses the same codec
  const int32_t* q;           // routed weight words [E, N, K/8] (NVFP4: the same bytes, [E, N, K/2] uint8)
  const uint16_t* s;          // routed scales (bytes of the codec's scale layout)
  const float* gsc;           // NVFP4: global scale per routed weight row [E, N]
  int N, K;                   // routed weight rows and reduction length
  const int32_t* q_sh;        // shared expert [N_sh, K_sh/8] (NVFP4: bytes [N_sh, K_sh/2]), null = none
  const uint16_t* s_sh;       // its scales in the codec's layout
  const float* gsc_sh;        // NVFP4: global scale per shared weight row [N_sh]
  int N_sh, K_sh;
  const int4* chunks;         // (expert, first position, rows, 0)
  const int* num_chunks;      // device count of valid chunks
  int max_chunks;             // chunk list capacity (grid size)
  int n_shared_chunks;        // ceil(T / chunk_rows) when the shared expert runs
  int chunk_rows;             // rows per chunk: 16 * kRowBlocks, or 16 (chunk_rows_for)
  int nslab;                  // column slabs per chunk
  uint16_t* h;                // gate_up output, routed rows [P, N/2]
  uint16_t* h_sh;             // gate_up output, shared rows [T, N_sh/2]
  int16_t* slots;             // down output codes [T, nslots, N] (block-permuted columns)
  float* slot_scale;          // down output scales [T, nslots, N / kSlotBlock]
  int nslots;                 // top_k, plus one when the shared expert runs
  const float* route_w;       // down: routing weight per assignment id [A]
  const float* gamma;         // down: shared-expert weight per token [T], null = 1
};

// Scheduler words of the persistent launch, zero before it (the align launch clears them): 8 ticket counters, 8 ready
// counters (one per queue), one done counter per chunk, then per queue (up to 8, each ceil(chunks / queues) long) the
// list of its chunks whose gate_up units have all finished, in the order they finished (chunk + 1; 0: not yet; kept
// by the 16-row tile's launch).
constexpr int kSchedWordsFixed = 16;
constexpr int kReadyWord = 8;
__host__ __device__ inline int sched_words(int max_chunks, int n_shared_chunks) {
  return kSchedWordsFixed + 2 * (max_chunks + n_shared_chunks) + 8;
}
constexpr int kNotFused = 1;  // launch_experts_fused: no persistent kernel for these sizes (or JANUS_MOE_SCHEDULE=split)

// gate_up then down in one persistent launch (sched: sched_words() ints, zero; status: the device status word, which
// gets kStatusGaveUp if a wait gave up); kNotFused when it does not apply.
int launch_experts_fused(const GemmParams& gu, const GemmParams& dn, int* sched, int* status, hipStream_t stream);
int launch_gate_up(const GemmParams& p, hipStream_t stream);
int launch_down(const GemmParams& p, hipStream_t stream);
// out[t, n] = bf16(sum_{j < nslots} slot value (t, j, n)), summed in slot order in fp32; 0 where valid[t] == 0 (valid
// null: every token). ids (null: none) are the top-k ids [T, topk]: a slot j < topk whose id is outside [0, E) is
// skipped.
int launch_combine(const int16_t* slots, const float* slot_scale, int nslots, uint16_t* out, int T, int H,
                   const uint8_t* valid, const int64_t* ids, int topk, int E, hipStream_t stream);
int launch_dequant(const int32_t* q, const uint16_t* s, long rows, int K, uint16_t* out, hipStream_t stream);
int launch_dequant_nvfp4(const uint8_t* q, const uint8_t* s, const float* gs, long rows, int K, uint16_t* out,
                         hipStream_t stream);

}  // namespace janus
