// Token-to-expert sort / align / permute on gfx950: a bit-exact integer restatement of align()
// (janus/moe_w4a16.py:89-106) in three launches, none of which reads back to the host:
//   1. rank    per block of 1024 assignments: an LDS histogram and the stable rank of every assignment among the
//              block's assignments of the same expert (wave ballots over the expert-id bits give the peers of each
//              lane; waves take their turn in assignment order);
//   2. scan    one workgroup: per-expert totals, per-(block, expert) offsets, padded expert starts, then either the
//              reference tile plan (expert_ids, total) or the GEMM chunk list;
//   3. scatter every assignment a lands at start[e] + offset[block][e] + rank[a].
// The stable order is the assignment id order, exactly as torch.argsort(stable=True) in the reference.
#include "align.h"

namespace janus {

namespace {

constexpr int kRankThreads = 256;
constexpr int kScanThreads = 1024;

// Inclusive scan of one int per thread over a 1024-thread block.
__device__ int block_inclusive_scan(int v, int* lds_waves /*[16]*/) {
  const int lane = lane_id(), wave = threadIdx.x / kWave;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    int o = __shfl_up(v, d);
    if (lane >= d) v += o;
  }
  if (lane == kWave - 1) lds_waves[wave] = v;
  __syncthreads();
  if (wave == 0) {
    int w = lane < (int)(blockDim.x / kWave) ? lds_waves[lane] : 0;
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) {
      int o = __shfl_up(w, d);
      if (lane >= d) w += o;
    }
    if (lane < 16) lds_waves[lane] = w;
  }
  __syncthreads();
  int r = v + (wave > 0 ? lds_waves[wave - 1] : 0);
  __syncthreads();
  return r;
}

template <typename IdxT, typename OutT>
__global__ void __launch_bounds__(kRankThreads) align_rank_kernel(const IdxT* __restrict__ idx, int A, int E, int nbits,
                                                                  int* __restrict__ hist, int* __restrict__ local_rank,
                                                                  OutT* __restrict__ sorted_ids, int sorted_len,
                                                                  float* __restrict__ zero_buf, long zero_len) {
  __shared__ int cnt[kMaxExperts];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  // Side jobs, grid-stride: fill the output permutation with the sentinel, clear the combine accumulator.
  for (long i = (long)blockIdx.x * blockDim.x + tid; i < sorted_len; i += (long)gridDim.x * blockDim.x)
    sorted_ids[i] = (OutT)A;
  if (zero_buf) {
    float4* z = reinterpret_cast<float4*>(zero_buf);
    for (long i = (long)blockIdx.x * blockDim.x + tid; i < zero_len / 4; i += (long)gridDim.x * blockDim.x)
      z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int base = blockIdx.x * kAlignChunk;
  if (base >= A) return;
  for (int e = tid; e < E; e += kRankThreads) cnt[e] = 0;
  __syncthreads();
  for (int round = 0; round < kAlignChunk / kRankThreads; ++round) {
    const int a = base + round * kRankThreads + tid;
    int e = -1;
    if (a < A) {
      long v = (long)idx[a];
      e = (v >= 0 && v < E) ? (int)v : -1;  // out-of-range ids are dropped
    }
    // Peers: lanes of this wave holding the same expert id.
    uint64_t peers = ballot(e >= 0);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = e >= 0 && ((e >> b) & 1);
      const uint64_t m = ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
    const int rank_in_wave = __popcll(peers & below);
    const int n_peers = __popcll(peers);
    const int leader = peers ? (__ffsll((unsigned long long)peers) - 1) : lane;
    // Waves of this round take their turn in assignment order.
    for (int w = 0; w < kRankThreads / kWave; ++w) {
      if (wave == w) {
        int start = 0;
        if (e >= 0 && lane == leader) {
          start = cnt[e];
          cnt[e] = start + n_peers;
        }
        start = __shfl(start, leader);
        if (e >= 0) local_rank[a] = start + rank_in_wave;
      }
      __syncthreads();
    }
  }
  for (int e = tid; e < E; e += kRankThreads) hist[(long)blockIdx.x * E + e] = cnt[e];
}

// One workgroup. hist [nb][E] becomes the exclusive per-expert prefix over blocks. `block` is the padding unit.
// Reference plan mode (expert_ids != null): expert_ids[i] = #{e : cum[e] <= i*block} (torch.searchsorted right=True
// over the inclusive padded cumsum), total[0] = cum[E-1]. Chunk mode (chunks != null): every expert's rows cut into
// runs of at most `chunk_rows`.
template <typename OutT>
__global__ void __launch_bounds__(kScanThreads) align_scan_kernel(int* __restrict__ hist, int nb, int E, int block,
                                                                  int* __restrict__ counts, int* __restrict__ start,
                                                                  OutT* __restrict__ expert_ids, int tiles,
                                                                  OutT* __restrict__ total_out, int4* __restrict__ chunks,
                                                                  int chunk_rows, int* __restrict__ num_chunks) {
  __shared__ int cum[kMaxExperts];
  __shared__ int waves[16];
  const int tid = threadIdx.x;
  int c = 0;
  if (tid < E) {
    for (int b = 0; b < nb; ++b) {
      const int h = hist[(long)b * E + tid];
      hist[(long)b * E + tid] = c;
      c += h;
    }
    counts[tid] = c;
  }
  const int padded = (c + block - 1) / block * block;
  const int incl = block_inclusive_scan(tid < E ? padded : 0, waves);
  if (tid < E) {
    cum[tid] = incl;
    start[tid] = incl - padded;
  }
  __syncthreads();
  const int total = cum[E - 1];
  if (expert_ids) {
    for (int i = tid; i < tiles; i += kScanThreads) {
      const long key = (long)i * block;
      int lo = 0, hi = E;  // first e with cum[e] > key
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((long)cum[mid] <= key) lo = mid + 1; else hi = mid;
      }
      expert_ids[i] = (OutT)lo;
    }
    if (tid == 0) total_out[0] = (OutT)total;
  }
  if (chunks) {
    const int nch = (c + chunk_rows - 1) / chunk_rows;
    const int incl_ch = block_inclusive_scan(tid < E ? nch : 0, waves);
    if (tid < E) {
      const int first = incl_ch - nch;
      for (int j = 0; j < nch; ++j)
        chunks[first + j] = make_int4(tid, start[tid] + j * chunk_rows, min(chunk_rows, c - j * chunk_rows), 0);
      if (tid == E - 1) num_chunks[0] = incl_ch;
    }
    if (E == 0 && tid == 0) num_chunks[0] = 0;
  }
}

template <typename IdxT, typename OutT>
__global__ void __launch_bounds__(kRankThreads) align_scatter_kernel(const IdxT* __restrict__ idx, int A, int E,
                                                                     const int* __restrict__ hist,
                                                                     const int* __restrict__ local_rank,
                                                                     const int* __restrict__ start,
                                                                     OutT* __restrict__ sorted_ids) {
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < kAlignChunk; i += kRankThreads) {
    const int a = b * kAlignChunk + i;
    if (a >= A) break;
    const long v = (long)idx[a];
    if (v < 0 || v >= E) continue;
    const int e = (int)v;
    sorted_ids[start[e] + hist[(long)b * E + e] + local_rank[a]] = (OutT)a;
  }
}

int expert_bits(int E) {
  int b = 0;
  while ((1 << b) < E) ++b;
  return b;
}

}  // namespace

AlignWorkspace carve_align(Carver& c, int A, int E) {
  AlignWorkspace w;
  const int nb = ceil_div(A, kAlignChunk);
  w.hist = c.take<int>((size_t)(nb > 0 ? nb : 1) * E);
  w.local_rank = c.take<int>(A > 0 ? A : 1);
  w.counts = c.take<int>(E);
  w.start = c.take<int>(E);
  return w;
}

template <typename IdxT, typename OutT>
int launch_align(const IdxT* idx, int A, int E, int block, const AlignWorkspace& w, OutT* sorted_ids, int sorted_len,
                 OutT* expert_ids, int tiles, OutT* total, int4* chunks, int chunk_rows, int* num_chunks,
                 float* zero_buf, long zero_len, hipStream_t stream) {
  const int nb = ceil_div(A, kAlignChunk);
  int grid = nb > 0 ? nb : 1;
  const int fill_blocks = ceil_div(sorted_len, kRankThreads * 8);
  if (fill_blocks > grid) grid = fill_blocks;
  const long zero_blocks = (zero_len / 4 + kRankThreads * 8 - 1) / (kRankThreads * 8);
  if (zero_blocks > grid) grid = (int)(zero_blocks < 4096 ? zero_blocks : 4096);
  hipLaunchKernelGGL((align_rank_kernel<IdxT, OutT>), dim3(grid), dim3(kRankThreads), 0, stream, idx, A, E,
                     expert_bits(E), w.hist, w.local_rank, sorted_ids, sorted_len, zero_buf, zero_len);
  JANUS_LAUNCH_CHECK("align_rank");
  hipLaunchKernelGGL((align_scan_kernel<OutT>), dim3(1), dim3(kScanThreads), 0, stream, w.hist, nb, E, block, w.counts,
                     w.start, expert_ids, tiles, total, chunks, chunk_rows, num_chunks);
  JANUS_LAUNCH_CHECK("align_scan");
  if (nb > 0) {
    hipLaunchKernelGGL((align_scatter_kernel<IdxT, OutT>), dim3(nb), dim3(kRankThreads), 0, stream, idx, A, E, w.hist,
                       w.local_rank, w.start, sorted_ids);
    JANUS_LAUNCH_CHECK("align_scatter");
  }
  return JANUS_MOE_OK;
}

template int launch_align<int64_t, int64_t>(const int64_t*, int, int, int, const AlignWorkspace&, int64_t*, int,
                                            int64_t*, int, int64_t*, int4*, int, int*, float*, long, hipStream_t);
template int launch_align<int64_t, int>(const int64_t*, int, int, int, const AlignWorkspace&, int*, int, int*, int,
                                        int*, int4*, int, int*, float*, long, hipStream_t);
template int launch_align<int, int>(const int*, int, int, int, const AlignWorkspace&, int*, int, int*, int, int*,
                                    int4*, int, int*, float*, long, hipStream_t);

}  // namespace janus

using namespace janus;

extern "C" size_t janus_moe_align_workspace_bytes(int S, int top_k, int E) {
  if (S < 0 || top_k <= 0 || E <= 0) return 0;
  Carver c(nullptr);
  carve_align(c, S * top_k, E);
  return align_up(c.used, 256);
}

extern "C" int janus_moe_align(const int64_t* top_k_index, int S, int top_k, int E, int block, int64_t* sorted_ids,
                               int64_t* expert_ids, int64_t* total, void* ws, size_t ws_bytes, janus_stream_t stream) {
  JANUS_REQUIRE(S >= 0 && top_k > 0 && E > 0 && E <= kMaxExperts && block > 0, JANUS_MOE_EINVAL,
                "janus_moe_align: unsupported sizes S=%d top_k=%d E=%d block=%d (need E <= %d)", S, top_k, E, block,
                kMaxExperts);
  const long A = (long)S * top_k;
  JANUS_REQUIRE(A < (1l << 30), JANUS_MOE_EINVAL, "janus_moe_align: S*top_k=%ld too large", A);
  JANUS_REQUIRE((A == 0 || top_k_index) && sorted_ids && expert_ids && total, JANUS_MOE_EINVAL,
                "janus_moe_align: null pointer");
  const size_t need = janus_moe_align_workspace_bytes(S, top_k, E);
  JANUS_REQUIRE(ws_bytes >= need && ws, JANUS_MOE_EWORKSPACE, "janus_moe_align: workspace %zu < %zu bytes", ws_bytes,
                need);
  Carver c(ws);
  AlignWorkspace w = carve_align(c, (int)A, E);
  const long tiles = (A + (long)E * (block - 1) + block - 1) / block;
  return launch_align<int64_t, int64_t>(top_k_index, (int)A, E, block, w, sorted_ids, (int)(tiles * block), expert_ids,
                                        (int)tiles, total, nullptr, 0, nullptr, nullptr, 0, (hipStream_t)stream);
}
