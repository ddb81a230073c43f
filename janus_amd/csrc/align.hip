// Token-to-expert sort / align / permute on gfx950: a bit-exact integer restatement of align()
// (janus/moe_w4a16.py:89-106). The stable order is the assignment id order, exactly as torch.argsort(stable=True) in
// the reference. Three schedules, chosen by size, with the same results:
//   one launch (A <= 32768 assignments: every batch up to 4K tokens at top-8): blocks of 256 assignments, each
//     workgroup counting all assignments per expert itself (LDS histograms) and placing its block;
//   small (A <= 65536): blocks of 256 assignments, two launches (rank, place), every block recomputing the
//     per-expert prefix it needs from the blocks' histograms;
//   large: blocks of 1024 assignments, three launches: rank (an LDS histogram and the stable rank of every assignment
//     among the block's assignments of the same expert, the block's waves taking their turn in order), scan (one
//     workgroup: per-expert totals, per-(block, expert) offsets, padded starts), scatter.
// Within a wave, the peers of a lane (lanes with the same expert id) come from wave ballots over the expert-id bits.
// Both schedules end with either the reference tile plan (expert_ids, total) or the GEMM chunk list.
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

// Peers of this lane (the lanes of its wave holding the same valid expert id e; none for e < 0): the lane's stable
// rank among them, their number and the lowest of them.
struct Peers {
  int rank, count, leader;
};
__device__ __forceinline__ Peers wave_peers(int e, int nbits) {
  const int lane = lane_id();
  uint64_t peers = ballot(e >= 0);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = e >= 0 && ((e >> b) & 1);
    const uint64_t m = ballot(bit);
    peers &= bit ? m : ~m;
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  Peers r;
  r.rank = __popcll(peers & below);
  r.count = __popcll(peers);
  r.leader = peers ? (int)__builtin_ctzll(peers) : lane;
  return r;
}

// The plan outputs from the inclusive padded cumsum cum[E] (LDS) and the padded starts: reference plan mode
// (expert_ids != null): expert_ids[i] = #{e : cum[e] <= i*block} (torch.searchsorted right=True), total[0] =
// cum[E-1]; chunk mode (chunks != null): every expert's rows cut into runs of at most `chunk_rows`. Thread tid < E
// holds expert tid's count and start. Called by every thread of the workgroup.
template <typename OutT>
__device__ void write_plan(const int* cum, int E, int block, int count, int start, OutT* expert_ids, int tiles,
                           OutT* total_out, int4* chunks, int chunk_rows, int* num_chunks, int* scan_tmp,
                           int* clear, int clear_n) {
  const int tid = threadIdx.x, nthreads = blockDim.x;
  for (int i = tid; i < clear_n; i += nthreads) clear[i] = 0;
  if (expert_ids) {
    for (int i = tid; i < tiles; i += nthreads) {
      const long key = (long)i * block;
      int lo = 0, hi = E;  // first e with cum[e] > key
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((long)cum[mid] <= key) lo = mid + 1; else hi = mid;
      }
      expert_ids[i] = (OutT)lo;
    }
    if (tid == 0) total_out[0] = (OutT)(E > 0 ? cum[E - 1] : 0);
  }
  if (chunks) {
    const int nch = tid < E ? (count + chunk_rows - 1) / chunk_rows : 0;
    const int incl_ch = block_inclusive_scan(nch, scan_tmp);
    if (tid < E) {
      const int first = incl_ch - nch;
      for (int j = 0; j < nch; ++j)
        chunks[first + j] = make_int4(tid, start + j * chunk_rows, min(chunk_rows, count - j * chunk_rows), 0);
      if (tid == E - 1) num_chunks[0] = incl_ch;
    }
    if (E == 0 && tid == 0) num_chunks[0] = 0;
  }
}

// The small schedule, A <= kSmallMaxA, two launches over blocks of kSmallBlock assignments.
//   align_small_rank:  per block, each wave's peers (wave ballots), the block's per-expert counts hist[b][e] and the
//                      rank of every assignment among the block's assignments of the same expert (local_rank);
//   align_small_place: every block recomputes each expert's total, padded start and the counts of the blocks before
//                      it from hist (nb <= 256 rows), then places its own assignments at start[e] + (assignments of e
//                      in earlier blocks) + local_rank; block 0 also writes the sentinel A at every padding position
//                      and past the last expert, and the plan outputs.
// No single-workgroup stage: the ranking and the scatter spread over nb workgroups.
constexpr int kSmallBlock = 256;
constexpr int kSmallWaves = kSmallBlock / kWave;
constexpr int kSmallMaxA = kSmallBlock * 256;
constexpr int kPlaceThreads = 1024;  // one thread per expert (E <= kMaxExperts)

// An assignment whose expert id is outside [0, E) is dropped; with `status` non-null it also sets kStatusDroppedIds
// there (the masked block routes padding tokens to id E on purpose and passes null).
__device__ __forceinline__ void report_dropped(int* status, bool dropped) {
  if (status && dropped) __hip_atomic_fetch_or(status, kStatusDroppedIds, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename IdxT>
__global__ void __launch_bounds__(kSmallBlock) align_small_rank_kernel(const IdxT* __restrict__ idx, int A, int E,
                                                                       int nbits, int* __restrict__ hist,
                                                                       int* __restrict__ local_rank,
                                                                       int* __restrict__ status) {
  __shared__ int wcnt[kSmallWaves][kMaxExperts];  // per-wave counts, then per-wave offsets within the block
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int a = blockIdx.x * kSmallBlock + tid;
  int e = -1;
  if (a < A) {
    const long v = (long)idx[a];
    e = (v >= 0 && v < E) ? (int)v : -1;  // out-of-range ids are dropped
    report_dropped(status, e < 0);
  }
  const Peers pr = wave_peers(e, nbits);
  for (int i = tid; i < kSmallWaves * kMaxExperts; i += kSmallBlock) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  if (e >= 0 && lane == pr.leader) wcnt[wave][e] = pr.count;
  __syncthreads();
  for (int x = tid; x < E; x += kSmallBlock) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < kSmallWaves; ++w) {
      const int h = wcnt[w][x];
      wcnt[w][x] = c;
      c += h;
    }
    hist[(long)blockIdx.x * E + x] = c;
  }
  __syncthreads();
  if (e >= 0) local_rank[a] = wcnt[wave][e] + pr.rank;
}

template <typename IdxT, typename OutT>
__global__ void __launch_bounds__(kPlaceThreads) align_small_place_kernel(
    const IdxT* __restrict__ idx, int A, int E, int block, int nb, const int* __restrict__ hist,
    const int* __restrict__ local_rank, OutT* __restrict__ sorted_ids, int sorted_len, OutT* __restrict__ expert_ids,
    int tiles, OutT* __restrict__ total_out, int4* __restrict__ chunks, int chunk_rows, int* __restrict__ num_chunks,
    int* __restrict__ clear, int clear_n) {
  __shared__ int cum[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int part_count[kPlaceThreads], part_before[kPlaceThreads];
  __shared__ int scan_tmp[16];
  const int tid = threadIdx.x, b = blockIdx.x;
  // Thread g E + x (g < G = kPlaceThreads / E groups) sums hist[j][x] over its blocks j = g mod G, eight loads in
  // flight at a time: all of the block's threads share the reads, and a read costs a fraction of a memory latency.
  const int G = kPlaceThreads / E;
  if (tid < G * E) {
    const int g = tid / E, x = tid - g * E;
    int pc = 0, pb = 0;
    for (int j0 = g; j0 < nb; j0 += 8 * G) {
      int h[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u * G;
        h[u] = hist[(long)(j < nb ? j : nb - 1) * E + x];  // no branch: a row past nb re-reads the last, dropped below
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (j0 + u * G >= nb) h[u] = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        pc += h[u];
        if (j0 + u * G < b) pb += h[u];
      }
    }
    part_count[tid] = pc;
    part_before[tid] = pb;
  }
  __syncthreads();
  int count = 0, before = 0;
  if (tid < E) {
    for (int g = 0; g < G; ++g) {
      count += part_count[g * E + tid];
      before += part_before[g * E + tid];
    }
  }
  const int padded = (count + block - 1) / block * block;
  const int incl = block_inclusive_scan(tid < E ? padded : 0, scan_tmp);
  const int start = incl - padded;
  if (tid < E) {
    cum[tid] = incl;
    base[tid] = start + before;
  }
  __syncthreads();
  if (tid < kSmallBlock) {
    const int a = b * kSmallBlock + tid;
    if (a < A) {
      const long v = (long)idx[a];
      if (v >= 0 && v < E) sorted_ids[base[(int)v] + local_rank[a]] = (OutT)a;
    }
  }
  if (b == 0) {
    if (tid < E)
      for (int i = count; i < padded; ++i) sorted_ids[start + i] = (OutT)A;
    const int total = E > 0 ? cum[E - 1] : 0;
    for (int i = total + tid; i < sorted_len; i += kPlaceThreads) sorted_ids[i] = (OutT)A;
    write_plan<OutT>(cum, E, block, count, start, expert_ids, tiles, total_out, chunks, chunk_rows, num_chunks,
                     scan_tmp, clear, clear_n);
  }
}

// Up to kOneMaxA assignments the small schedule's two launches are one: every workgroup also counts all A
// assignments per expert (and those before its block) in LDS, from the expert ids themselves, in place of the
// per-block histograms the second launch would read. Each workgroup reads all of idx (64 KB at 16K assignments, from
// the L2), which is what bounds the size. The results are those of the two launches.
constexpr int kOneMaxA = 32768;

template <typename IdxT, typename OutT>
__global__ void __launch_bounds__(kPlaceThreads) align_one_kernel(
    const IdxT* __restrict__ idx, int A, int E, int nbits, int block, OutT* __restrict__ sorted_ids, int sorted_len,
    OutT* __restrict__ expert_ids, int tiles, OutT* __restrict__ total_out, int4* __restrict__ chunks,
    int chunk_rows, int* __restrict__ num_chunks, int* __restrict__ clear, int clear_n, int* __restrict__ status) {
  __shared__ int all_c[kMaxExperts], before_c[kMaxExperts];
  __shared__ int wcnt[kSmallWaves][kMaxExperts];  // per-wave counts of the block, then per-wave offsets
  __shared__ int cum[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int scan_tmp[16];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave, b = blockIdx.x;
  const int a0 = b * kSmallBlock;
  for (int i = tid; i < kMaxExperts; i += kPlaceThreads) {
    all_c[i] = 0;
    before_c[i] = 0;
  }
  for (int i = tid; i < kSmallWaves * kMaxExperts; i += kPlaceThreads) (&wcnt[0][0])[i] = 0;
  // this block's own assignment, loaded together with the first pass below
  int e = -1;
  const int a = a0 + tid;
  if (tid < kSmallBlock && a < A) {
    const long v = (long)idx[a];
    e = (v >= 0 && v < E) ? (int)v : -1;
    report_dropped(status, e < 0);
  }
  __syncthreads();
  // every assignment, sixteen loads in flight per thread (one pass up to 16K assignments). The loads take no branch
  // (an index past A re-reads the last id, dropped afterwards): a load under a branch would be waited for at once.
  constexpr int kLoads = 16;
  for (int i0 = tid; i0 < A; i0 += kLoads * kPlaceThreads) {
    long v[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int i = i0 + u * kPlaceThreads;
      v[u] = (long)idx[i < A ? i : A - 1];
    }
#pragma unroll
    for (int u = 0; u < kLoads; ++u)
      if (i0 + u * kPlaceThreads >= A) v[u] = -1;
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      if (v[u] >= 0 && v[u] < E) {
        atomicAdd(&all_c[(int)v[u]], 1);
        if (i0 + u * kPlaceThreads < a0) atomicAdd(&before_c[(int)v[u]], 1);
      }
    }
  }
  // stable rank of the block's assignments among the block's assignments of the same expert (as align_small_rank)
  Peers pr = {0, 0, 0};
  if (tid < kSmallBlock) {  // whole waves
    pr = wave_peers(e, nbits);
    if (e >= 0 && lane == pr.leader) wcnt[wave][e] = pr.count;
  }
  __syncthreads();
  if (tid < E) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < kSmallWaves; ++w) {
      const int h = wcnt[w][tid];
      wcnt[w][tid] = c;
      c += h;
    }
  }
  const int count = tid < E ? all_c[tid] : 0;
  const int padded = (count + block - 1) / block * block;
  const int incl = block_inclusive_scan(tid < E ? padded : 0, scan_tmp);  // its barriers order the wcnt offsets too
  const int start = incl - padded;
  if (tid < E) {
    cum[tid] = incl;
    base[tid] = start + before_c[tid];
  }
  __syncthreads();
  if (e >= 0) sorted_ids[base[e] + wcnt[wave][e] + pr.rank] = (OutT)a;
  if (b == 0) {
    if (tid < E)
      for (int i = count; i < padded; ++i) sorted_ids[start + i] = (OutT)A;
    const int total = E > 0 ? cum[E - 1] : 0;
    for (int i = total + tid; i < sorted_len; i += kPlaceThreads) sorted_ids[i] = (OutT)A;
    write_plan<OutT>(cum, E, block, count, start, expert_ids, tiles, total_out, chunks, chunk_rows, num_chunks,
                     scan_tmp, clear, clear_n);
  }
}

template <typename IdxT, typename OutT>
__global__ void __launch_bounds__(kRankThreads) align_rank_kernel(const IdxT* __restrict__ idx, int A, int E, int nbits,
                                                                  int* __restrict__ hist, int* __restrict__ local_rank,
                                                                  OutT* __restrict__ sorted_ids, int sorted_len,
                                                                  int* __restrict__ status) {
  __shared__ int cnt[kMaxExperts];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  // Side job, grid-stride: fill the output permutation with the sentinel.
  for (long i = (long)blockIdx.x * blockDim.x + tid; i < sorted_len; i += (long)gridDim.x * blockDim.x)
    sorted_ids[i] = (OutT)A;
  const int base = blockIdx.x * kAlignChunk;
  if (base >= A) return;
  for (int e = tid; e < E; e += kRankThreads) cnt[e] = 0;
  // the block's ids, loaded together before the passes below store ranks (an index past A re-reads the last id;
  // dropped): a load after a possibly aliasing store, or under a branch, would cost a memory round trip each
  constexpr int kPasses = kAlignChunk / kRankThreads;
  long ids[kPasses];
#pragma unroll
  for (int r = 0; r < kPasses; ++r) {
    const int a = base + r * kRankThreads + tid;
    ids[r] = (long)idx[a < A ? a : A - 1];
  }
  __syncthreads();
#pragma unroll
  for (int round = 0; round < kPasses; ++round) {
    const int a = base + round * kRankThreads + tid;
    const long v = ids[round];
    const int e = (a < A && v >= 0 && v < E) ? (int)v : -1;  // out-of-range ids are dropped
    report_dropped(status, a < A && e < 0);
    const Peers pr = wave_peers(e, nbits);
    const int rank_in_wave = pr.rank, n_peers = pr.count, leader = pr.leader;
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
                                                                  int chunk_rows, int* __restrict__ num_chunks,
                                                                  int* __restrict__ clear, int clear_n) {
  __shared__ int cum[kMaxExperts];
  __shared__ int waves[16];
  const int tid = threadIdx.x;
  // sixteen blocks' counts loaded together, then overwritten with the running offsets: a load written after a store
  // into the same array waits for the loads before it, one memory round trip per block (a row past nb re-reads the
  // last row, before any store of the batch; dropped)
  constexpr int kBatch = 16;
  int c = 0;
  if (tid < E) {
    for (int b0 = 0; b0 < nb; b0 += kBatch) {
      int h[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) h[u] = hist[(long)(b0 + u < nb ? b0 + u : nb - 1) * E + tid];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (b0 + u < nb) {
          hist[(long)(b0 + u) * E + tid] = c;
          c += h[u];
        }
      }
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
  write_plan<OutT>(cum, E, block, c, tid < E ? start[tid] : 0, expert_ids, tiles, total_out, chunks, chunk_rows,
                   num_chunks, waves, clear, clear_n);
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
  const int nb = A <= kSmallMaxA ? ceil_div(A, kSmallBlock) : ceil_div(A, kAlignChunk);
  w.hist = c.take<int>((size_t)(nb > 0 ? nb : 1) * E);
  w.local_rank = c.take<int>(A > 0 ? A : 1);
  w.counts = c.take<int>(E);
  w.start = c.take<int>(E);
  return w;
}

namespace {
// First index in [lo, hi) whose value is >= key, for values non-decreasing over [lo, hi).
__device__ int lower_bound64(const int64_t* __restrict__ v, int lo, int hi, int64_t key) {
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (v[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// The GEMM chunk list from a caller's reference tile plan (align() at any block size): thread e finds expert e's
// tiles by binary search over expert_ids (non-decreasing; tiles past the total hold ids >= E) and its real rows by
// binary search for the first sentinel in them (real assignment ids come first), then cuts those rows into chunks.
// The permutation is copied as is (values outside [0, A] become the sentinel A), and clear[0 .. clear_n) is zeroed.
// A plan that does not come from align cannot make the GEMMs go out of bounds: chunks stay inside the plan's rows
// and the list's capacity, and the GEMMs skip rows whose id is not below A.
__global__ void __launch_bounds__(kScanThreads) plan_chunks_kernel(
    const int64_t* __restrict__ psorted, const int64_t* __restrict__ pexpert, int tiles, int block, int A, int E,
    int* __restrict__ sorted_ids, int4* __restrict__ chunks, int capacity, int chunk_rows, int* __restrict__ num_chunks,
    int* __restrict__ clear, int clear_n) {
  __shared__ int waves[16];
  const int tid = threadIdx.x;
  const int P = tiles * block;
  for (int i = tid; i < P; i += blockDim.x) {
    const int64_t v = psorted[i];
    sorted_ids[i] = (v >= 0 && v < A) ? (int)v : A;
  }
  for (int i = tid; i < clear_n; i += blockDim.x) clear[i] = 0;
  int start = 0, count = 0;
  if (tid < E) {
    const int lo = lower_bound64(pexpert, 0, tiles, tid), hi = lower_bound64(pexpert, lo, tiles, tid + 1);
    start = lo * block;
    // rows [start, start + count): the ids below A before the expert's first sentinel
    int a = start, b = hi * block;
    while (a < b) {
      const int mid = (a + b) >> 1;
      const int64_t v = psorted[mid];
      if (v >= 0 && v < A) a = mid + 1;
      else b = mid;
    }
    count = a - start;
  }
  const int nch = (count + chunk_rows - 1) / chunk_rows;
  const int end = block_inclusive_scan(nch, waves);
  for (int j = 0; j < nch; ++j) {
    const int at = end - nch + j;
    if (at < capacity) chunks[at] = make_int4(tid, start + j * chunk_rows, min(chunk_rows, count - j * chunk_rows), 0);
  }
  if (tid == (int)blockDim.x - 1) *num_chunks = min(end, capacity);
}
}  // namespace

int launch_plan_chunks(const int64_t* psorted, const int64_t* pexpert, int tiles, int block, int A, int E,
                       int* sorted_ids, int4* chunks, int capacity, int chunk_rows, int* num_chunks, int* clear,
                       int clear_n, hipStream_t stream) {
  JANUS_REQUIRE(E > 0 && E <= kScanThreads, JANUS_MOE_EINVAL, "plan chunks: E=%d (at most %d)", E, kScanThreads);
  hipLaunchKernelGGL(plan_chunks_kernel, dim3(1), dim3(kScanThreads), 0, stream, psorted, pexpert, tiles, block, A, E,
                     sorted_ids, chunks, capacity, chunk_rows, num_chunks, clear, clear_n);
  JANUS_LAUNCH_CHECK("plan_chunks");
  return JANUS_MOE_OK;
}

template <typename IdxT, typename OutT>
int launch_align(const IdxT* idx, int A, int E, int block, const AlignWorkspace& w, OutT* sorted_ids, int sorted_len,
                 OutT* expert_ids, int tiles, OutT* total, int4* chunks, int chunk_rows, int* num_chunks,
                 int* clear, int clear_n, int* status, hipStream_t stream) {
  if (A <= kOneMaxA) {
    hipLaunchKernelGGL((align_one_kernel<IdxT, OutT>), dim3(A > 0 ? ceil_div(A, kSmallBlock) : 1), dim3(kPlaceThreads),
                       0, stream, idx, A, E, expert_bits(E), block, sorted_ids, sorted_len, expert_ids, tiles, total,
                       chunks, chunk_rows, num_chunks, clear, clear_n, status);
    JANUS_LAUNCH_CHECK("align_one");
    return JANUS_MOE_OK;
  }
  if (A <= kSmallMaxA) {
    const int nb = ceil_div(A, kSmallBlock);
    if (nb > 0) {
      hipLaunchKernelGGL((align_small_rank_kernel<IdxT>), dim3(nb), dim3(kSmallBlock), 0, stream, idx, A, E,
                         expert_bits(E), w.hist, w.local_rank, status);
      JANUS_LAUNCH_CHECK("align_small_rank");
    }
    hipLaunchKernelGGL((align_small_place_kernel<IdxT, OutT>), dim3(nb > 0 ? nb : 1), dim3(kPlaceThreads), 0, stream,
                       idx, A, E, block, nb, w.hist, w.local_rank, sorted_ids, sorted_len, expert_ids, tiles, total,
                       chunks, chunk_rows, num_chunks, clear, clear_n);
    JANUS_LAUNCH_CHECK("align_small_place");
    return JANUS_MOE_OK;
  }
  const int nb = ceil_div(A, kAlignChunk);
  int grid = nb;
  const int fill_blocks = ceil_div(sorted_len, kRankThreads * 8);
  if (fill_blocks > grid) grid = fill_blocks;
  hipLaunchKernelGGL((align_rank_kernel<IdxT, OutT>), dim3(grid), dim3(kRankThreads), 0, stream, idx, A, E,
                     expert_bits(E), w.hist, w.local_rank, sorted_ids, sorted_len, status);
  JANUS_LAUNCH_CHECK("align_rank");
  hipLaunchKernelGGL((align_scan_kernel<OutT>), dim3(1), dim3(kScanThreads), 0, stream, w.hist, nb, E, block, w.counts,
                     w.start, expert_ids, tiles, total, chunks, chunk_rows, num_chunks, clear, clear_n);
  JANUS_LAUNCH_CHECK("align_scan");
  hipLaunchKernelGGL((align_scatter_kernel<IdxT, OutT>), dim3(nb), dim3(kRankThreads), 0, stream, idx, A, E, w.hist,
                     w.local_rank, w.start, sorted_ids);
  JANUS_LAUNCH_CHECK("align_scatter");
  return JANUS_MOE_OK;
}

template int launch_align<int64_t, int64_t>(const int64_t*, int, int, int, const AlignWorkspace&, int64_t*, int,
                                            int64_t*, int, int64_t*, int4*, int, int*, int*, int, int*, hipStream_t);
template int launch_align<int64_t, int>(const int64_t*, int, int, int, const AlignWorkspace&, int*, int, int*, int,
                                        int*, int4*, int, int*, int*, int, int*, hipStream_t);
template int launch_align<int, int>(const int*, int, int, int, const AlignWorkspace&, int*, int, int*, int, int*,
                                    int4*, int, int*, int*, int, int*, hipStream_t);

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
                                        (int)tiles, total, nullptr, 0, nullptr, nullptr, 0, device_status_word(),
                                        (hipStream_t)stream);
}
