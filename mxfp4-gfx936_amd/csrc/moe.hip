// Routed MoE on the device: routing metadata, the grouped-GEMM entry points,
// the top-k combine, and the whole vLLM MoE layer (vllm:233-265).
//
// Routing (the format of vllm:119-146, consumed as soft:101-108) is built
// without any host synchronisation in three deterministic passes over
// 1024-route chunks:
//   count  -- per-chunk expert histogram (LDS atomics; counts only);
//   scan   -- one workgroup turns the histograms into, for every (chunk,
//             expert), the absolute position of that chunk's first route of
//             that expert, pads every expert to block_m, writes expert_ids,
//             the sentinel padding and num_tokens_post_padded;
//   place  -- each chunk places its routes in route order: the rank of a
//             route among earlier same-expert routes of its wave comes from
//             ballots over the expert-id bits, across waves from a small
//             per-wave count table in LDS.
// The result is identical to the host loop of vllm:119-146 (ascending
// experts, ascending route ids inside an expert) for ids in [0, E); other ids
// are dropped, leaving those rows untouched (soft:476-481: they stay zero).
#include <algorithm>
#include <mutex>

#include "gemm.h"

namespace mx {
namespace {

constexpr int kChunk = 1024;  // routes per count/place workgroup
// Routes the single-workgroup routing handles: up to kSingle one 256-thread
// workgroup; up to kSingleWide one 1024-thread workgroup (4096 routes: ~6
// us in the kernel against 15.4 us of kernel time for the three launches;
// for up to 1024 routes, 256 threads beat 1024: 5.0 vs 5.4 us).
constexpr int kSingle = 1024;
constexpr int kSingleWide = 4096;
// Layers with at most this many routes use direct routing in the GEMMs
// (no kernel builds sorted metadata); must not exceed the skinny kernel's
// scan limit (256).
constexpr int64_t kDirectRoutes = 64;
constexpr int kMaxExperts = 1024;
// Experts the single-workgroup routing kernel holds in LDS (more use the
// three-launch path).
constexpr int kSingleExperts = 256;

// Expert of a route: its id when in [0, num_experts), else drop_to.  With
// drop_to = -1 the route is dropped (in no block; its output rows are not
// written).  The fused soft op passes num_experts = E + 1 and drop_to = E:
// dropped routes then gather in blocks of the extra expert E, which the
// GEMMs (experts outside [0, E) -> zeros) fill with zeros.
template <typename TI>
__device__ __forceinline__ int route_expert(TI id, int num_experts, int drop_to) {
  const int64_t e = (int64_t)id;
  return (e >= 0 && e < num_experts) ? (int)e : drop_to;
}

template <typename TI>
__global__ __launch_bounds__(256) void align_count(const TI* __restrict__ ids, int64_t n,
                                                   int num_experts, int drop_to,
                                                   int32_t* __restrict__ counts) {
  __shared__ int hist[kMaxExperts];
  for (int e = threadIdx.x; e < num_experts; e += 256) hist[e] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  for (int i = 0; i < kChunk / 256; ++i) {
    const int64_t r = base + i * 256 + threadIdx.x;
    if (r < n) {
      const int e = route_expert(ids[r], num_experts, drop_to);
      if (e >= 0) atomicAdd(&hist[e], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < num_experts; e += 256)
    counts[(int64_t)blockIdx.x * num_experts + e] = hist[e];
}

// One 1024-thread workgroup; thread e owns expert e.  Chunk counts are
// loaded kScanBatch at a time (one memory round trip each; the first
// batch's prefixes are kept in registers until the start is known), the padded
// expert totals are scanned with wave shuffles plus the 16 wave sums, and
// the sentinel padding and expert_ids are written by whole waves (an
// expert's padding is < block_m entries: at most two per lane).
constexpr int kScanBatch = 32;

__global__ __launch_bounds__(1024) void align_scan(int32_t* __restrict__ counts, int nchunks,
                                                   int num_experts, int block_m, int64_t n,
                                                   int32_t* __restrict__ sorted_ids,
                                                   int32_t* __restrict__ expert_ids,
                                                   int32_t* __restrict__ num_post_padded) {
  __shared__ int wsum[kMaxExperts / 64];
  __shared__ int s_start[kMaxExperts], s_total[kMaxExperts], s_pad[kMaxExperts];
  const int e = threadIdx.x;
  const int lane = e & 63, wave = e >> 6;
  // exclusive prefix over chunks within the expert; the first batch's
  // prefixes stay in registers, later batches go back to memory
  int total = 0;
  int pre[kScanBatch];
  if (e < num_experts) {
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j)
      pre[j] = j < nchunks ? counts[(int64_t)j * num_experts + e] : 0;
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) {
      const int c = pre[j];
      pre[j] = total;
      total += c;
    }
    for (int b0 = kScanBatch; b0 < nchunks; b0 += kScanBatch) {
      int c[kScanBatch];
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j)
        c[j] = b0 + j < nchunks ? counts[(int64_t)(b0 + j) * num_experts + e] : 0;
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j)
        if (b0 + j < nchunks) {
          counts[(int64_t)(b0 + j) * num_experts + e] = total;
          total += c[j];
        }
    }
  }
  const int padded = e < num_experts ? ((total + block_m - 1) / block_m) * block_m : 0;
  // inclusive scan of the padded totals over experts
  int v = padded;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off);
    if (lane >= off) v += u;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  for (int w = 0; w < wave; ++w) v += wsum[w];
  const int start = v - padded;  // exclusive
  if (e < num_experts) {
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j)
      if (j < nchunks) counts[(int64_t)j * num_experts + e] = pre[j] + start;
    for (int b0 = kScanBatch; b0 < nchunks; b0 += kScanBatch) {
      int c[kScanBatch];
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j)
        c[j] = b0 + j < nchunks ? counts[(int64_t)(b0 + j) * num_experts + e] : 0;
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j)
        if (b0 + j < nchunks) counts[(int64_t)(b0 + j) * num_experts + e] = c[j] + start;
    }
    s_start[e] = start;
    s_total[e] = total;
    s_pad[e] = padded;
  }
  if (e == num_experts - 1) num_post_padded[0] = v;
  __syncthreads();
  for (int x = wave; x < num_experts; x += kMaxExperts / 64) {
    const int st = s_start[x], end = st + s_pad[x];
    for (int i = lane; i < s_pad[x] / block_m; i += 64) expert_ids[st / block_m + i] = x;
    for (int p = st + s_total[x] + lane; p < end; p += 64) sorted_ids[p] = (int32_t)n;
  }
}

template <typename TI>
__global__ __launch_bounds__(256) void align_place(const TI* __restrict__ ids, int64_t n,
                                                   int num_experts, int drop_to, int id_bits,
                                                   const int32_t* __restrict__ starts,
                                                   int32_t* __restrict__ sorted_ids) {
  __shared__ int cursor[kMaxExperts];
  __shared__ int wcnt[4][kMaxExperts];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  for (int e = tid; e < num_experts; e += 256) {
    cursor[e] = starts[(int64_t)blockIdx.x * num_experts + e];
    wcnt[0][e] = wcnt[1][e] = wcnt[2][e] = wcnt[3][e] = 0;
  }
  __syncthreads();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  for (int it = 0; it < kChunk / 256; ++it) {
    const int64_t r = base + it * 256 + tid;
    const int em = r < n ? route_expert(ids[r], num_experts, drop_to) : -1;
    const bool valid = em >= 0;
    const int e = valid ? em : 0;
    uint64_t same = __ballot(valid);
    for (int bit = 0; bit < id_bits; ++bit) {
      const bool b = (e >> bit) & 1;
      const uint64_t bal = __ballot(b);
      same &= b ? bal : ~bal;
    }
    const int rank = __popcll(same & lt_mask);
    if (valid && rank == 0) wcnt[wave][e] = __popcll(same);
    __syncthreads();
    if (valid) {
      int before = cursor[e] + rank;
      for (int w = 0; w < wave; ++w) before += wcnt[w][e];
      sorted_ids[before] = (int32_t)r;
    }
    __syncthreads();
    for (int x = tid; x < num_experts; x += 256) {
      cursor[x] += wcnt[0][x] + wcnt[1][x] + wcnt[2][x] + wcnt[3][x];
      wcnt[0][x] = wcnt[1][x] = wcnt[2][x] = wcnt[3][x] = 0;
    }
    __syncthreads();
  }
}

// Scan and placement in one launch, after align_count, for at most
// kScanPlaceChunks chunks: workgroup c places chunk c's kChunk routes and
// first derives what it needs from the per-chunk counts itself -- for each
// expert the routes of the earlier chunks and of all chunks (coalesced
// loads, summed with LDS atomics), the padded exclusive scan over the
// experts -- instead of waiting for a separate scan launch (redundant work
// of nchunks x E count loads per workgroup, all L2 hits).  Placement as in
// align_single: wave w owns routes w * RPT * 64 .. +RPT * 64 of the chunk,
// the lanes of a sub-chunk with the same expert come from ballots, per-wave
// counts become per-wave positions, and each wave then places its
// sub-chunks in order without barriers.  Workgroup c also writes, by whole
// waves, expert_ids and the sentinel padding of the experts x with x %
// nchunks == c, and workgroup 0 the padded route count.
constexpr int kScanPlaceChunks = 64;

template <typename TI>
__global__ __launch_bounds__(512) void align_scan_place(const TI* __restrict__ ids, int64_t n,
                                                        int num_experts, int drop_to,
                                                        int id_bits, int block_m,
                                                        const int32_t* __restrict__ counts,
                                                        int nchunks,
                                                        int32_t* __restrict__ sorted_ids,
                                                        int32_t* __restrict__ expert_ids,
                                                        int32_t* __restrict__ num_post_padded) {
  constexpr int NT = 512, W = NT / 64, RPT = kChunk / NT;
  constexpr int EPT = kMaxExperts / NT;  // experts per thread in the scan
  constexpr int CB = 16;                 // count loads per thread per round trip
  __shared__ int wpos[W * kMaxExperts];  // [wave][expert]: counts, then next positions
  __shared__ int s_pre[kMaxExperts], s_tot[kMaxExperts];  // then fill start / padded end
  __shared__ int part[W];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = (int)blockIdx.x;
  const int ne = num_experts;
  int eid[RPT];
  const int64_t rbase = (int64_t)c * kChunk + (int64_t)wave * (RPT * 64);
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int64_t r = rbase + j * 64 + lane;
    eid[j] = r < n ? route_expert(ids[r], ne, drop_to) : -1;
  }
  const int ncnt = nchunks * ne;
  int cv[CB];
#pragma unroll
  for (int b = 0; b < CB; ++b) cv[b] = tid + b * NT < ncnt ? counts[tid + b * NT] : 0;
  for (int i = tid; i < W * ne; i += NT) wpos[i] = 0;
  for (int x = tid; x < ne; x += NT) s_pre[x] = s_tot[x] = 0;
  __syncthreads();
  // counts[cc][x] -> routes of expert x in all chunks and in chunks < c
  // (i / ne by a float reciprocal and one correction: i < 2^16)
  const float inv_ne = 1.0f / (float)ne;
  for (int i0 = 0; i0 < ncnt; i0 += CB * NT) {
    if (i0 > 0) {
#pragma unroll
      for (int b = 0; b < CB; ++b)
        cv[b] = i0 + tid + b * NT < ncnt ? counts[i0 + tid + b * NT] : 0;
    }
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      const int i = i0 + tid + b * NT;
      if (i < ncnt && cv[b] != 0) {
        int cc = (int)((float)i * inv_ne);
        cc += (cc + 1) * ne <= i ? 1 : 0;
        cc -= cc * ne > i ? 1 : 0;
        const int x = i - cc * ne;
        atomicAdd(&s_tot[x], cv[b]);
        if (cc < c) atomicAdd(&s_pre[x], cv[b]);
      }
    }
  }
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint64_t same[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) same[j] = __ballot(eid[j] >= 0);
  for (int bit = 0; bit < id_bits; ++bit) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const bool b = (eid[j] >> bit) & 1;  // lanes of invalid ids are out of every mask
      const uint64_t bal = __ballot(b);
      same[j] &= b ? bal : ~bal;
    }
  }
#pragma unroll
  for (int j = 0; j < RPT; ++j)
    if (eid[j] >= 0 && __popcll(same[j] & lt_mask) == 0)
      wpos[wave * ne + eid[j]] += __popcll(same[j]);
  __syncthreads();
  // padded exclusive scan over the experts (thread-local EPT, wave
  // shuffles, then the wave sums)
  int tot[EPT], pad[EPT], local = 0;
#pragma unroll
  for (int jj = 0; jj < EPT; ++jj) {
    const int x = tid * EPT + jj;
    tot[jj] = x < ne ? s_tot[x] : 0;
    pad[jj] = (tot[jj] + block_m - 1) / block_m * block_m;
    local += pad[jj];
  }
  int v = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off);
    if (lane >= off) v += u;
  }
  if (lane == 63) part[wave] = v;
  __syncthreads();
  for (int w = 0; w < wave; ++w) v += part[w];
  int start = v - local;
#pragma unroll
  for (int jj = 0; jj < EPT; ++jj) {
    const int x = tid * EPT + jj;
    if (x < ne) {
      int p = start + s_pre[x];
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const int cw = wpos[w * ne + x];
        wpos[w * ne + x] = p;
        p += cw;
      }
      s_pre[x] = start;           // now: first slot of the expert
      s_tot[x] = start + tot[jj];  // now: first sentinel slot
    }
    start += pad[jj];
  }
  if (c == 0 && tid == NT - 1) num_post_padded[0] = v;
  __syncthreads();
  // expert ids and sentinel padding of this workgroup's experts, by waves
  for (int x = c + wave * nchunks; x < ne; x += W * nchunks) {
    const int st = s_pre[x], fill = s_tot[x];
    const int end = fill == st ? st : st + (fill - st + block_m - 1) / block_m * block_m;
    for (int i = lane; i < (end - st) / block_m; i += 64) expert_ids[st / block_m + i] = x;
    for (int q = fill + lane; q < end; q += 64) sorted_ids[q] = (int32_t)n;
  }
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    if (rbase + j * 64 >= n) break;  // the same for the whole wave
    if (eid[j] >= 0) {
      const int e = eid[j];
      const int rank = __popcll(same[j] & lt_mask);
      const int base = wpos[wave * ne + e];
      sorted_ids[base + rank] = (int32_t)(rbase + j * 64 + lane);
      if (rank == 0) wpos[wave * ne + e] = base + __popcll(same[j]);
    }
  }
}

// out[t, :] = sum over slots s of d[t * top_k + s, :] (FP32, slot order),
// skipping slots whose expert id is outside [0, E) (their rows are zero in
// the reference, soft:476).  vllm:263-265.
template <typename T, typename TI>
__global__ __launch_bounds__(256) void topk_sum(const T* __restrict__ d, const TI* __restrict__ ids,
                                                int64_t m, int top_k, int64_t hidden,
                                                int num_experts, T* __restrict__ out) {
  typedef typename Decode<T>::vec8 V8;
  const int64_t vecs = hidden >> 3;
  const int64_t total = m * vecs;
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < total;
       u += (int64_t)gridDim.x * 256) {
    const int64_t t = u / vecs;
    const int64_t c = (u - t * vecs) * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // eight slots per step, all loads issued before the first add (slots
    // past top_k re-read the last one and are masked); the adds keep slot
    // order
    for (int s0 = 0; s0 < top_k; s0 += 8) {
      V8 v[8];
      bool ok[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int s = s0 + q < top_k ? s0 + q : top_k - 1;
        const int64_t e = (int64_t)ids[t * top_k + s];
        ok[q] = (s0 + q < top_k) && e >= 0 && e < num_experts;
        v[q] = *reinterpret_cast<const V8*>(d + (t * top_k + s) * hidden + c);
      }
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (ok[q]) {
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] += (float)v[q][j];
        }
    }
    V8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = from_f32<T>(acc[j]);
    *reinterpret_cast<V8*>(out + t * hidden + c) = o;
  }
}

// All three passes in one workgroup of NT threads for at most NT * RPT
// routes and kSingleExperts experts (decode and small prefill).  Wave w owns
// routes w * RPT * 64 .. +RPT * 64 in RPT sub-chunks of 64, so route order
// is wave, then sub-chunk, then lane.  (1) Each lane finds the lanes of its
// sub-chunk with the same expert (one ballot per id bit; the masks are kept
// for step 3) and the lowest of them adds their count to the wave's row of
// per-expert counts.  (2) One thread per expert sums its wave counts, the
// padded sizes are scanned over the experts, and the wave rows become each
// wave's first position per expert; expert ids and sentinel padding are
// written.  (3) Every route lands at its wave's position for its expert +
// its rank among the lower lanes, and the lowest lane advances the position
// for the next sub-chunk -- route order within an expert, as align_place.
// Three barriers in all (the placement needs none: a wave's LDS accesses
// are ordered); 4096 routes: 9.1 -> 5.9 us, 1024: 7.7 -> 5.0 us of
// in-kernel time against per-chunk placement over the whole workgroup.
// When the padded routing fits kStageIds entries, the sentinel fill and the
// placement write an LDS copy of sorted_ids, which then goes out in
// coalesced stores instead of scattered ones (two more barriers; graph
// replays of the call, 4096 routes over 129 experts: 7.16 -> 6.42 us, 1024
// routes: 5.41 -> 4.94 us).
constexpr int kStageIds = 12288;
template <typename TI, int NT, int RPT>
__global__ __launch_bounds__(NT) void align_single(const TI* __restrict__ ids, int64_t n,
                                                   int num_experts, int drop_to, int id_bits,
                                                   int block_m,
                                                   int32_t* __restrict__ sorted_ids,
                                                   int32_t* __restrict__ expert_ids,
                                                   int32_t* __restrict__ num_post_padded) {
  constexpr int W = NT / 64;                // waves
  constexpr int E = kSingleExperts;
  constexpr int EPT = (E + NT - 1) / NT;    // experts per thread in the scan
  __shared__ int wpos[W][E];                // per-wave counts, then next positions
  __shared__ int part[W];
  __shared__ int s_fill[E], s_end[E];       // first sentinel slot, end of the padded range
  __shared__ int s_total;
  __shared__ int32_t s_ids[kStageIds];      // staged sorted_ids (padded total <= kStageIds)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int eid[RPT];
  const int64_t rbase = (int64_t)wave * (RPT * 64);
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int64_t r = rbase + j * 64 + lane;
    eid[j] = r < n ? route_expert(ids[r], num_experts, drop_to) : -1;
  }
  for (int i = tid; i < W * E; i += NT) (&wpos[0][0])[i] = 0;
  __syncthreads();
  // (1) lanes of the sub-chunk with the same expert; the RPT ballot chains
  // are independent, so they are interleaved bit by bit
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint64_t same[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) same[j] = __ballot(eid[j] >= 0);
  for (int bit = 0; bit < id_bits; ++bit) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const bool b = (eid[j] >> bit) & 1;  // lanes of invalid ids are out of every mask
      const uint64_t bal = __ballot(b);
      same[j] &= b ? bal : ~bal;
    }
  }
#pragma unroll
  for (int j = 0; j < RPT; ++j)
    if (eid[j] >= 0 && __popcll(same[j] & lt_mask) == 0) wpos[wave][eid[j]] += __popcll(same[j]);
  __syncthreads();
  // (2) padded exclusive scan: thread tid owns experts tid*EPT .. +EPT; the
  // per-thread totals are scanned with wave shuffles, then the wave sums
  int cnt[EPT], pad[EPT], local = 0;
#pragma unroll
  for (int jj = 0; jj < EPT; ++jj) {
    const int x = tid * EPT + jj;
    int c = 0;
    if (x < num_experts) {
      int cw[W];  // all reads first: one LDS round trip, not W
#pragma unroll
      for (int w = 0; w < W; ++w) cw[w] = wpos[w][x];
#pragma unroll
      for (int w = 0; w < W; ++w) c += cw[w];
    }
    cnt[jj] = c;
    pad[jj] = (c + block_m - 1) / block_m * block_m;
    local += pad[jj];
  }
  int v = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off);
    if (lane >= off) v += u;
  }
  if (lane == 63) part[wave] = v;
  __syncthreads();
  for (int w = 0; w < wave; ++w) v += part[w];
  int start = v - local;
#pragma unroll
  for (int jj = 0; jj < EPT; ++jj) {
    const int x = tid * EPT + jj;
    if (x < num_experts) {
      int p = start;
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const int c = wpos[w][x];
        wpos[w][x] = p;
        p += c;
      }
      for (int blk = start / block_m; blk < (start + pad[jj]) / block_m; ++blk) expert_ids[blk] = x;
      s_fill[x] = start + cnt[jj];
      s_end[x] = start + pad[jj];
    }
    start += pad[jj];
  }
  if (tid == NT - 1) {
    num_post_padded[0] = v;
    s_total = v;
  }
  __syncthreads();
  const int total = s_total;
  if (total <= kStageIds) {
    for (int i = tid; i < total; i += NT) s_ids[i] = (int32_t)n;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      if (rbase + j * 64 >= n) break;  // the same for the whole wave
      if (eid[j] >= 0) {
        const int e = eid[j];
        const int rank = __popcll(same[j] & lt_mask);
        const int base = wpos[wave][e];
        s_ids[base + rank] = (int32_t)(rbase + j * 64 + lane);
        if (rank == 0) wpos[wave][e] = base + __popcll(same[j]);
      }
    }
    __syncthreads();
    for (int i = tid; i < total; i += NT) sorted_ids[i] = s_ids[i];
    return;
  }
  // sentinel padding (at most block_m - 1 slots per expert): consecutive
  // lanes on consecutive slots of one expert
  if ((block_m & (block_m - 1)) == 0) {
    const int sh = __builtin_ctz(block_m);
    for (int i = tid; i < num_experts * block_m; i += NT) {
      const int x = i >> sh;
      const int q = s_fill[x] + (i & (block_m - 1));
      if (q < s_end[x]) sorted_ids[q] = (int32_t)n;
    }
  } else {
    for (int i = tid; i < num_experts * block_m; i += NT) {
      const int x = i / block_m;
      const int q = s_fill[x] + (i - x * block_m);
      if (q < s_end[x]) sorted_ids[q] = (int32_t)n;
    }
  }
  // (3) placement
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    if (rbase + j * 64 >= n) break;  // the same for the whole wave
    if (eid[j] >= 0) {
      const int e = eid[j];
      const int rank = __popcll(same[j] & lt_mask);
      const int base = wpos[wave][e];
      sorted_ids[base + rank] = (int32_t)(rbase + j * 64 + lane);
      if (rank == 0) wpos[wave][e] = base + __popcll(same[j]);
    }
  }
}

int64_t round_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

void align_capacity(int64_t n, int num_experts, int block_m, int64_t* max_sorted,
                    int64_t* max_blocks, int64_t* nchunks) {
  const int64_t busy = n < num_experts ? n : num_experts;
  const int64_t cap = round_up(n + busy * (block_m - 1), block_m);
  *max_sorted = cap > 0 ? cap : block_m;
  *max_blocks = *max_sorted / block_m;
  *nchunks = (n + kChunk - 1) / kChunk;
}

int check_align_args(int64_t n, int num_experts, int block_m, int ids_dtype) {
  if (ids_dtype != MXFP4_DT_I32 && ids_dtype != MXFP4_DT_I64) {
    set_error("topk_ids must be int32 or int64");
    return MXFP4_ERR_TYPE;
  }
  if (n < 0 || num_experts < 1 || num_experts > kMaxExperts || block_m < 16 || block_m % 16 ||
      n > (int64_t)0x3FFFFFFF) {
    set_error("routing: unsupported sizes (routes %lld, experts %d, block_m %d)", (long long)n,
              num_experts, block_m);
    return MXFP4_ERR_VALUE;
  }
  return MXFP4_OK;
}

template <typename TI>
int launch_align(const TI* ids, int64_t n, int num_experts, int drop_to, int block_m,
                 int32_t* sorted_ids, int32_t* expert_ids, int32_t* npp, int32_t* counts,
                 int64_t nchunks, hipStream_t st) {
  int id_bits = 0;
  while ((1 << id_bits) < num_experts) ++id_bits;
  const bool single = num_experts <= kSingleExperts;
  if (single && n <= kSingle) {
    align_single<TI, 256, kSingle / 256><<<1, 256, 0, st>>>(
        ids, n, num_experts, drop_to, id_bits, block_m, sorted_ids, expert_ids, npp);
    return launch_status("align launch");
  }
  if (single && n <= kSingleWide) {
    align_single<TI, 1024, kSingleWide / 1024><<<1, 1024, 0, st>>>(
        ids, n, num_experts, drop_to, id_bits, block_m, sorted_ids, expert_ids, npp);
    return launch_status("align launch");
  }
  if (nchunks > 0) {
    align_count<TI><<<(unsigned)nchunks, 256, 0, st>>>(ids, n, num_experts, drop_to, counts);
    int rc = launch_status("align count launch");
    if (rc) return rc;
  }
  if (nchunks > 0 && nchunks <= kScanPlaceChunks) {
    align_scan_place<TI><<<(unsigned)nchunks, 512, 0, st>>>(ids, n, num_experts, drop_to, id_bits,
                                                             block_m, counts, (int)nchunks,
                                                             sorted_ids, expert_ids, npp);
    return launch_status("align scan+place launch");
  }
  align_scan<<<1, kMaxExperts, 0, st>>>(counts, (int)nchunks, num_experts, block_m, n, sorted_ids,
                                        expert_ids, npp);
  int rc = launch_status("align scan launch");
  if (rc) return rc;
  if (nchunks > 0) {
    align_place<TI><<<(unsigned)nchunks, 256, 0, st>>>(ids, n, num_experts, drop_to, id_bits,
                                                       counts, sorted_ids);
    rc = launch_status("align place launch");
  }
  return rc;
}

// drop_to: -1 (routes of ids outside [0, num_experts) are dropped) or
// num_experts - 1 (they gather in that last expert's blocks).
int do_align(const void* ids, int ids_dtype, int64_t n, int num_experts, int block_m,
             int32_t* sorted_ids, int32_t* expert_ids, int32_t* npp, int32_t* counts,
             int64_t nchunks, hipStream_t st, int drop_to = -1) {
  if (ids_dtype == MXFP4_DT_I32)
    return launch_align(static_cast<const int32_t*>(ids), n, num_experts, drop_to, block_m,
                        sorted_ids, expert_ids, npp, counts, nchunks, st);
  return launch_align(static_cast<const int64_t*>(ids), n, num_experts, drop_to, block_m,
                      sorted_ids, expert_ids, npp, counts, nchunks, st);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int dispatch_gemm(const GemmArgs& g, int a_dtype, int c_dtype, int epi, hipStream_t st) {
  if (a_dtype == MXFP4_DT_U8 || a_dtype == MXFP4_DT_F8E4M3 || a_dtype == MXFP4_DT_F8E5M2) {
    if (epi != EPI_STORE) {
      set_error("packed / FP8 activations support the plain epilogue only");
      return MXFP4_ERR_VALUE;
    }
    GemmArgs g8 = g;
    g8.a_fp8 = a_dtype == MXFP4_DT_F8E4M3 ? 1 : (a_dtype == MXFP4_DT_F8E5M2 ? 2 : 0);
    return launch_w4a4(g8, c_dtype, st);
  }
  if (c_dtype == MXFP4_DT_F32) {
    if (epi != EPI_STORE) {
      set_error("the FP32 compute path supports the plain epilogue only");
      return MXFP4_ERR_TYPE;
    }
    // bf16 A on routed blocks of 32k rows: the bf16 MFMA's products of A and
    // the E2M1 x 2^k weights (exact in bf16) are exact and summed in FP32,
    // the FP32 GEMM's arithmetic up to the summation order; the W4A16 prefill
    // tiles then store FP32.  Other A types and block sizes: the FP32 MFMA.
    if (a_dtype == MXFP4_DT_BF16 && g.sorted_ids && !g.route_ids && g.block_m % 32 == 0 &&
        pf_supported(g, 2))
      return launch_w4a16(g, MXFP4_DT_BF16, EPI_STORE_F32, st);
    return launch_f32_reference(g, a_dtype, st);
  }
  if (a_dtype != c_dtype) {
    set_error("activation dtype %d must equal the compute dtype %d", a_dtype, c_dtype);
    return MXFP4_ERR_TYPE;
  }
  return launch_w4a16(g, c_dtype, epi, st);
}

int64_t elem_size(int dt) {
  switch (dt) {
    case MXFP4_DT_F32: case MXFP4_DT_I32: return 4;
    case MXFP4_DT_BF16: case MXFP4_DT_F16: return 2;
    case MXFP4_DT_I64: return 8;
    default: return 1;
  }
}

struct LayerPlan {
  int block_m;
  int64_t routes, max_sorted, max_blocks, nchunks;
  int64_t off_counts, off_sorted, off_experts, off_npp, off_h, off_d, total;
};

LayerPlan plan_layer(int64_t m, int top_k, int num_experts, int64_t hidden, int64_t inter,
                     int64_t esize, bool prepacked) {
  LayerPlan p;
  p.routes = m * top_k;
  const double avg = (double)p.routes / (double)num_experts;
  // routing block per average routes per expert (MoE layer, 128 experts,
  // top-8, prepacked, steady clocks): 16-row blocks up to ~1.5 routes per
  // expert, 32 (32 x 256 tiles) up to ~32, 64 (64 x 256 tiles) above.
  // E.g. 96 tokens 93.6 us with 16 vs 78.4 us with 32; 448 tokens 102.3 us
  // with 64 vs 96.6 us with 32; 640 tokens 112.3 us with 64 vs 117.3 us
  // with 32 (re-measured with the register epilogues, 3 weight copies
  // rotated, 32 vs 64 rows: 448 / 512 / 576 tokens 95.1 / 96.3 / 121.0 vs
  // 98.7 / 101.0 / 104.2 us).  Against 128-row blocks (persistent 128 x 256 tiles, whose
  // fixed rounds of 512 workgroups quantize): 2048 tokens 236 -> 224 us,
  // 4096 385 -> 372 us, 6144 559 -> 521 us, 16384 1289 -> 1283 us; 128 rows
  // win only where their tiles just fill whole rounds (1536 tokens 166 vs
  // 182 us, 1664 170 vs 184 us).
  p.block_m = avg <= 1.5 ? 16 : (avg <= 32.0 ? 32 : 64);
  // Checkpoint-layout weights (no prepacked copies) take the fused soft
  // op's rule -- 32-row blocks up to 28 routes per expert, 64 up to 56,
  // 128 above -- with BM x 128 SiLU tiles on 32- and 64-row blocks and
  // 128 x 256 on 128-row ones (pf_choose).  Layer, graph replays (E=128,
  // top-8, H=2048, I=768): 256 tokens 112.0 -> 108.8 us, 512 153.2 ->
  // 126.1, 1024 185.5 -> 160.2, 2048 246.7 -> 242.5, 4096 418.2 -> 414.4.
  // With the weight-line groups of the checkpoint tiles, 16-row blocks (the
  // single-trip decode kernels) win up to 6 routes per expert (layer, graph
  // replays over 3 weight copies, 32 / 48 / 64 / 96 tokens: 82.2 / 85.4 /
  // 88.4 / 94.8 vs 92.1 / 93.4 / 97.2 / 98.5 us with 32 rows; the
  // prepacked layer keeps 32 rows: 75.0-78.1 vs 82.2-94.8 us).
  if (!prepacked) p.block_m = avg <= 6.0 ? 16 : (avg <= 28.0 ? 32 : (avg <= 56.0 ? 64 : 128));
  align_capacity(p.routes, num_experts, p.block_m, &p.max_sorted, &p.max_blocks, &p.nchunks);
  int64_t off = 0;
  p.off_counts = off; off = round_up(off + (p.nchunks > 0 ? p.nchunks : 1) * num_experts * 4, 256);
  p.off_sorted = off; off = round_up(off + p.max_sorted * 4, 256);
  p.off_experts = off; off = round_up(off + p.max_blocks * 4, 256);
  p.off_npp = off; off = round_up(off + 4, 256);
  p.off_h = off; off = round_up(off + p.routes * inter * esize, 256);
  p.off_d = off; off = round_up(off + p.routes * hidden * esize, 256);
  p.total = off;
  return p;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mxfp4_moe_align_sizes(int64_t num_routes, int num_experts, int block_m,
                                     int64_t* max_sorted, int64_t* max_blocks,
                                     int64_t* align_workspace_bytes) {
  int rc = check_align_args(num_routes, num_experts, block_m, MXFP4_DT_I64);
  if (rc) return rc;
  int64_t nchunks;
  align_capacity(num_routes, num_experts, block_m, max_sorted, max_blocks, &nchunks);
  *align_workspace_bytes = (nchunks > 0 ? nchunks : 1) * num_experts * 4;
  return MXFP4_OK;
}

extern "C" int mxfp4_moe_align(const void* topk_ids, int ids_dtype, int64_t num_routes,
                               int num_experts, int block_m, int32_t* sorted_ids,
                               int32_t* expert_ids, int32_t* num_post_padded, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  int rc = check_align_args(num_routes, num_experts, block_m, ids_dtype);
  if (rc) return rc;
  int64_t ms, mb, nchunks;
  align_capacity(num_routes, num_experts, block_m, &ms, &mb, &nchunks);
  if (workspace_bytes < (nchunks > 0 ? nchunks : 1) * num_experts * 4) {
    set_error("routing workspace too small");
    return MXFP4_ERR_VALUE;
  }
  return do_align(topk_ids, ids_dtype, num_routes, num_experts, block_m, sorted_ids, expert_ids,
                  num_post_padded, static_cast<int32_t*>(workspace), nchunks,
                  static_cast<hipStream_t>(stream));
}

namespace mx {
namespace {

// Checks shared by the routed GEMM entry points (mxfp4_moe_gemm,
// mxfp4_fused_moe); em / block_m are the metadata capacity and block size.
int check_routed_args(const void* a, int a_dtype, int64_t a_row_stride, const uint8_t* a_mx,
                      const uint8_t* b, int64_t num_experts, int64_t n, int64_t k, int c_dtype,
                      int top_k, int block_m, int64_t em) {
  if (c_dtype != MXFP4_DT_BF16 && c_dtype != MXFP4_DT_F16 && c_dtype != MXFP4_DT_F32) {
    set_error("unsupported software fallback compute dtype: %d", c_dtype);
    return MXFP4_ERR_TYPE;
  }
  if (a_dtype == MXFP4_DT_U8 && a_mx == nullptr) {
    set_error("packed MXFP4 activations require A_mx_scale");
    return MXFP4_ERR_VALUE;
  }
  if (a_dtype != MXFP4_DT_U8 && a_dtype != MXFP4_DT_F8E4M3 && a_dtype != MXFP4_DT_F8E5M2 &&
      a_dtype != MXFP4_DT_F32 && a_dtype != MXFP4_DT_BF16 && a_dtype != MXFP4_DT_F16) {
    set_error("unsupported activation dtype %d", a_dtype);
    return MXFP4_ERR_TYPE;
  }
  if (k <= 0 || k % 32 != 0 || n <= 0 || n > 0x7FFFFFFF || k > 0x7FFFFFFF || num_experts < 1 ||
      top_k < 1 || block_m < 16 || block_m % 16 != 0 || em < 0 || em % block_m != 0) {
    set_error("moe gemm: invalid sizes (n %lld, k %lld, block_m %d, em %lld)", (long long)n,
              (long long)k, block_m, (long long)em);
    return MXFP4_ERR_VALUE;
  }
  if (!aligned16(a) || !aligned16(b) || (a_row_stride * elem_size(a_dtype)) % 16) {
    set_error("moe gemm: activation/weight rows must be 16-byte aligned");
    return MXFP4_ERR_VALUE;
  }
  return MXFP4_OK;
}

GemmArgs routed_args(const void* a, int64_t a_rows, int64_t a_row_stride, const uint8_t* a_mx,
                     const uint8_t* b, const uint8_t* b_mx, int64_t num_experts, int64_t n,
                     int64_t k, void* c, int64_t c_row_stride, const float* a_scale,
                     const float* b_scale, const float* topk_weights, int mul_routed_weight,
                     const int32_t* sorted_ids, const int32_t* expert_ids,
                     const int32_t* num_post_padded, int64_t em, int block_m, int64_t num_valid,
                     int top_k) {
  GemmArgs g = {};
  g.a = a;
  g.a_mx = a_mx;
  g.a_rows = a_rows;
  g.lda = a_row_stride;
  g.lda_mx = k / 32;
  g.b = b;
  g.bs = b_mx;
  g.b_n = k / 2;
  g.b_e = n * (k / 2);
  g.bs_n = k / 32;
  g.bs_e = n * (k / 32);
  g.c = c;
  g.ldc = c_row_stride;
  g.sorted_ids = sorted_ids;
  g.expert_ids = expert_ids;
  g.num_post_padded = num_post_padded;
  g.a_scale = a_scale;
  g.b_scale = b_scale;
  // mul_routed_weight bit 0: multiply the route weights; bit 1: the
  // reference safe path's rounding sequence (ref_scaled)
  g.route_w = (mul_routed_weight & 1) ? topk_weights : nullptr;
  g.ref_round = (mul_routed_weight >> 1) & 1;
  g.m = em;
  g.num_valid = num_valid;
  g.n = (int32_t)n;
  g.k = (int32_t)k;
  g.top_k = top_k;
  g.block_m = block_m;
  g.num_experts = (int32_t)num_experts;
  return g;
}

// Rows per expert block of the fused soft op.  Its weights come in the
// checkpoint layout, where a prefill tile stages 32 bytes of every weight
// row per 64-deep step (one cache line per row), so blocks of more rows
// amortize the weight loads better than on the prepacked layout.  W4A16,
// E=128, top-8, routed GEMM alone, graph replays (MI355X; K=2048 N=1536 /
// K=768 N=2048 per routes per expert): 16 -> 32-row blocks 51.6 / 28.4 us
// (64 rows: 54.6 / 33.2); 32 -> 64 rows 59.0 / 35.9 (32 rows: 67.7 /
// 35.1); 48 -> 64 rows 66.2 / 41.3 (128: 76.5 / 47.1); 64 -> 128 rows
// 80.2 / 52.3 (64: 84.0 / 49.3); 256 -> 128 rows 235.9 / 146.5 (64: 235.8 /
// 151.0).  The W4A4 path keeps the 16 / 32 / 64 rule.  The FP32 path
// (f32_pipe, MFMA bound, skipping row blocks of padding only): 16 rows up to
// 8 routes per expert, else 32 (AITER's entry on the same routes, K=2048
// N=1536: 4 routes per expert 153.6 / 163.9 / 221.7 us for 16 / 32 / 64;
// 32: 366.0 / 337.7 / 374.2; 128: 1219 / 1048 / 1107).
enum SoftPath {
  SOFT_W4A16,      // bf16 / fp16 A and C, checkpoint-layout weights
  SOFT_W4A16_PRE,  // the same with a prepacked copy
  SOFT_SCALED,     // packed MXFP4 / FP8 A on the block-scaled MFMA
  SOFT_F32,        // C in FP32, fp16 / fp32 A (FP32 MFMA)
  SOFT_F32_W4A16,  // C in FP32, bf16 A: the W4A16 prefill tiles storing FP32
  SOFT_F32_W4A16_PRE,
};

SoftPath soft_path(int a_dtype, int c_dtype, bool prepacked) {
  if (a_dtype == MXFP4_DT_U8 || a_dtype == MXFP4_DT_F8E4M3 || a_dtype == MXFP4_DT_F8E5M2)
    return SOFT_SCALED;
  if (c_dtype == MXFP4_DT_F32) {
    if (a_dtype != MXFP4_DT_BF16) return SOFT_F32;
    return prepacked ? SOFT_F32_W4A16_PRE : SOFT_F32_W4A16;
  }
  return prepacked ? SOFT_W4A16_PRE : SOFT_W4A16;
}

// With a prepacked copy (AITER's entry on the copy, E=128, top-8, 32 vs
// 64-row blocks, 16 / 24 / 32 / 48 routes per expert; us): 32 rows up to 16
// routes per expert, 64 above 32, and between the two 64 where K >= 2048
// (longer K streams more weight bytes per padded row): N=1536 K=2048 40.1 /
// 43.9 / 50.7 / 50.8 vs 42.8 / 44.0 / 44.6 / 47.2; N=1024 K=4096 52.0 /
// 67.4 / 65.7 / 78.2 vs 55.8 / 59.3 / 61.6 / 65.4; N=3072 K=2048 83.7 /
// 106.7 / 108.7 / 113.0 vs 94.6 / 98.1 / 100.0 / 107.0; N=2048 K=3072 91.2
// / 114.0 / 106.0 / 141.6 vs 105.9 / 108.7 / 113.0 / 119.2; N=2048 K=768
// 23.1 / 27.3 / 27.5 / 35.7 vs 29.9 / 30.5 / 31.2 / 33.8; N=4096 K=1024
// 75.0 / 73.4 / 73.4 / 91.7 vs 73.9 / 76.9 / 79.4 / 88.1.  The packed /
// FP8 path keeps 32 up to 32 routes per expert, else 64.
int soft_block_m(int64_t routes, int64_t num_experts, SoftPath path, int64_t k) {
  if (path == SOFT_F32_W4A16 || path == SOFT_F32_W4A16_PRE) {
    // the W4A16 rule, at least 32 rows (the prefill tiles); on the
    // checkpoint layout 32 rows up to 32 routes per expert (C in FP32 moves
    // twice the output bytes: the soft op at 512 tokens, 32 routes per
    // expert, 81 us on 32-row blocks against 90 us on 64)
    const double avg = (double)routes / (double)(num_experts > 0 ? num_experts : 1);
    if (path == SOFT_F32_W4A16 && avg > 1.5 && avg <= 32.0) return 32;
    const int b = soft_block_m(routes, num_experts,
                               path == SOFT_F32_W4A16 ? SOFT_W4A16 : SOFT_W4A16_PRE, k);
    return b < 32 ? 32 : b;
  }
  const double avg = (double)routes / (double)(num_experts > 0 ? num_experts : 1);
  if (avg <= 1.5) return 16;
  if (path == SOFT_F32) return avg <= 8.0 ? 16 : 32;
  if (path == SOFT_W4A16_PRE) return avg <= 16.0 ? 32 : (avg > 32.0 || k >= 2048 ? 64 : 32);
  if (path == SOFT_SCALED) return avg <= 32.0 ? 32 : 64;
  // checkpoint layout, long K: 16-row blocks (the single-trip decode
  // kernels) up to 4 routes per expert (AITER's entry, graph replays,
  // K=2048 N=1536, 3 / 4 / 6 / 8 / 12 / 16 routes per expert, 16 vs 32
  // rows: 42.0 / 47.8 / 52.3 / 55.7 / 60.1 / 63.2 vs 45.2 / 56.6 / 58.1 /
  // 58.6 / 59.4 / 59.6 us; K=768 N=2048 takes 32 rows from 1.5 routes per
  // expert: 27.8 / 31.9 / 34.5 vs 24.1 / 27.3 / 29.4 at 3 / 4 / 6)
  if (k >= 2048 && avg <= 4.0) return 16;
  // checkpoint layout above 56 routes per expert: 128 rows only for long K
  // (AITER's entry, 64 / 128 / 256 routes per expert, 64 vs 128 rows: K=768
  // N=2048 46.8 / 75.5 / 130.9 vs 50.6 / 79.0 / 132.5 us; K=2048 N=1536
  // 84.1 / 129.7 / 235.6 vs 80.8 / 129.0 / 229.5)
  // (32 rows up to 32 routes per expert, 30 where K >= 2048: on cold
  // weights -- graph replays over 3 copies -- 32 vs 64 rows at 24 / 32 / 40
  // routes per expert: K=768 36.9 / 39.9 / 47.4 vs 40.1 / 40.7 / 42.3 us;
  // K=2048 with the register epilogues, at 20 / 24 / 28 / 32 / 36 routes:
  // 63.3 / 71.0 / 74.9 / 80.1 / 88.0 vs 74.9 / 76.7 / 77.6 / 78.5 / 81.0)
  return avg <= (k >= 2048 ? 30.0 : 32.0) ? 32 : (avg <= 56.0 || k < 2048 ? 64 : 128);
}

struct SoftPlan {
  int block_m;
  int align_experts;  // experts the routing counts (E + 1: dropped routes in the last)
  int drop_to;        // route_expert's target for ids outside [0, E)
  bool zero_c;        // E + 1 experts do not fit the routing: zero C first instead
  int64_t max_sorted, max_blocks, nchunks;
  int64_t off_counts, off_sorted, off_experts, off_npp, total;
};

SoftPlan plan_soft(int64_t routes, int64_t num_experts, SoftPath path, int64_t k) {
  SoftPlan p;
  p.block_m = soft_block_m(routes, num_experts, path, k);
  p.zero_c = num_experts + 1 > kMaxExperts;
  p.align_experts = (int)(p.zero_c ? num_experts : num_experts + 1);
  p.drop_to = p.zero_c ? -1 : (int)num_experts;
  align_capacity(routes, p.align_experts, p.block_m, &p.max_sorted, &p.max_blocks, &p.nchunks);
  int64_t off = 0;
  p.off_counts = off;
  off = round_up(off + (p.nchunks > 0 ? p.nchunks : 1) * p.align_experts * 4, 256);
  p.off_sorted = off; off = round_up(off + p.max_sorted * 4, 256);
  p.off_experts = off; off = round_up(off + p.max_blocks * 4, 256);
  p.off_npp = off; off = round_up(off + 4, 256);
  p.total = off;
  return p;
}

// The prepacked copy (prepack.hip) of the GEMM's experts x n x k weights,
// read by the W4A16 prefill kernels instead of b / bs (bitwise the same
// results); null pointers: none.
void set_prepacked(GemmArgs& g, const uint8_t* pre_b, const uint16_t* pre_s, int64_t n,
                   int64_t k) {
  g.pre_b = pre_b;
  g.pre_s = pre_s;
  g.pre_b_e = prepacked_nibble_bytes(n, k);
  g.pre_s_e = prepacked_scale_bytes(n, k);
}

// Zero `bytes` bytes at p (16-byte aligned; bytes % 2 == 0): a fill kernel,
// not hipMemsetAsync, so the call can be captured in a graph.
__global__ __launch_bounds__(256) void zero_fill(uint8_t* __restrict__ p, int64_t bytes) {
  const int64_t nv = bytes / 16;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < nv; i += stride)
    reinterpret_cast<i32x4*>(p)[i] = i32x4{0, 0, 0, 0};
  for (int64_t i = nv * 16 + blockIdx.x * 256 + threadIdx.x; i < bytes; i += stride) p[i] = 0;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mxfp4_moe_gemm(const void* a, int a_dtype, int64_t a_rows, int64_t a_row_stride,
                              const uint8_t* a_mx, const uint8_t* b, const uint8_t* b_mx,
                              int64_t num_experts, int64_t n, int64_t k, void* c, int c_dtype,
                              int64_t c_row_stride, const float* a_scale, const float* b_scale,
                              const float* topk_weights, int mul_routed_weight,
                              const int32_t* sorted_ids, const int32_t* expert_ids,
                              const int32_t* num_post_padded, int64_t em, int block_m,
                              int64_t num_valid, int top_k, void* stream) {
  return mxfp4_moe_gemm_pre(a, a_dtype, a_rows, a_row_stride, a_mx, b, b_mx, nullptr, nullptr,
                            num_experts, n, k, c, c_dtype, c_row_stride, a_scale, b_scale,
                            topk_weights, mul_routed_weight, sorted_ids, expert_ids,
                            num_post_padded, em, block_m, num_valid, top_k, stream);
}

extern "C" int mxfp4_moe_gemm_pre(const void* a, int a_dtype, int64_t a_rows,
                                  int64_t a_row_stride, const uint8_t* a_mx, const uint8_t* b,
                                  const uint8_t* b_mx, const uint8_t* pre_b, const uint16_t* pre_s,
                                  int64_t num_experts, int64_t n, int64_t k, void* c, int c_dtype,
                                  int64_t c_row_stride, const float* a_scale, const float* b_scale,
                                  const float* topk_weights, int mul_routed_weight,
                                  const int32_t* sorted_ids, const int32_t* expert_ids,
                                  const int32_t* num_post_padded, int64_t em, int block_m,
                                  int64_t num_valid, int top_k, void* stream) {
  int rc = check_routed_args(a, a_dtype, a_row_stride, a_mx, b, num_experts, n, k, c_dtype, top_k,
                             block_m, em);
  if (rc) return rc;
  if ((pre_b == nullptr) != (pre_s == nullptr)) {
    set_error("moe gemm: the prepacked nibbles and scales come together");
    return MXFP4_ERR_VALUE;
  }
  if (em == 0) return MXFP4_OK;
  GemmArgs g = routed_args(a, a_rows, a_row_stride, a_mx, b, b_mx, num_experts, n, k, c,
                           c_row_stride, a_scale, b_scale, topk_weights, mul_routed_weight,
                           sorted_ids, expert_ids, num_post_padded, em, block_m, num_valid, top_k);
  set_prepacked(g, pre_b, pre_s, n, k);
  return dispatch_gemm(g, a_dtype, c_dtype, EPI_STORE, static_cast<hipStream_t>(stream));
}

extern "C" int mxfp4_fused_moe_workspace_size(int64_t m, int top_k, int64_t num_experts,
                                              int a_dtype, int c_dtype, int64_t* bytes) {
  if (bytes == nullptr || m < 0 || top_k < 1 || num_experts < 1 || num_experts > kMaxExperts ||
      m * top_k > (int64_t)0x3FFFFFFF) {
    set_error("fused moe: invalid sizes (m %lld, top_k %d, experts %lld)", (long long)m, top_k,
              (long long)num_experts);
    return MXFP4_ERR_VALUE;
  }
  // every plan fits: either layout (the caller may pass a prepacked copy),
  // any K
  int64_t most = 0;
  for (int pre = 0; pre < 2; ++pre)
    for (int64_t k : {(int64_t)0, (int64_t)1 << 30}) {
      const int64_t t = plan_soft(m * top_k, num_experts, soft_path(a_dtype, c_dtype, pre), k).total;
      most = t > most ? t : most;
    }
  *bytes = most;
  return MXFP4_OK;
}

extern "C" int mxfp4_fused_moe(const void* a, int a_dtype, int64_t a_rows, int64_t a_row_stride,
                               const uint8_t* a_mx, const uint8_t* b, const uint8_t* b_mx,
                               int64_t num_experts, int64_t n, int64_t k, void* c, int c_dtype,
                               const float* a_scale, const float* b_scale,
                               const float* topk_weights, int mul_routed_weight,
                               const void* topk_ids, int ids_dtype, int64_t m, int top_k,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  return mxfp4_fused_moe_pre(a, a_dtype, a_rows, a_row_stride, a_mx, b, b_mx, nullptr, nullptr,
                             num_experts, n, k, c, c_dtype, a_scale, b_scale, topk_weights,
                             mul_routed_weight, topk_ids, ids_dtype, m, top_k, workspace,
                             workspace_bytes, stream);
}

extern "C" int mxfp4_fused_moe_pre(const void* a, int a_dtype, int64_t a_rows,
                                   int64_t a_row_stride, const uint8_t* a_mx, const uint8_t* b,
                                   const uint8_t* b_mx, const uint8_t* pre_b, const uint16_t* pre_s,
                                   int64_t num_experts, int64_t n, int64_t k, void* c, int c_dtype,
                                   const float* a_scale, const float* b_scale,
                                   const float* topk_weights, int mul_routed_weight,
                                   const void* topk_ids, int ids_dtype, int64_t m, int top_k,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  if (ids_dtype != MXFP4_DT_I32 && ids_dtype != MXFP4_DT_I64) {
    set_error("topk_ids must be int32 or int64");
    return MXFP4_ERR_TYPE;
  }
  if ((pre_b == nullptr) != (pre_s == nullptr)) {
    set_error("fused moe: the prepacked nibbles and scales come together");
    return MXFP4_ERR_VALUE;
  }
  if (m < 0 || m * (int64_t)(top_k > 0 ? top_k : 1) > (int64_t)0x3FFFFFFF ||
      num_experts > kMaxExperts) {
    set_error("fused moe: invalid sizes (m %lld, top_k %d, experts %lld)", (long long)m, top_k,
              (long long)num_experts);
    return MXFP4_ERR_VALUE;
  }
  const int64_t routes = m * top_k;
  const SoftPlan p =
      plan_soft(routes, num_experts, soft_path(a_dtype, c_dtype, pre_b != nullptr), k);
  int rc = check_routed_args(a, a_dtype, a_row_stride, a_mx, b, num_experts, n, k, c_dtype, top_k,
                             p.block_m, p.max_sorted);
  if (rc) return rc;
  if (!aligned16(c)) {
    set_error("fused moe: C must be 16-byte aligned");
    return MXFP4_ERR_VALUE;
  }
  if (workspace_bytes < p.total || (p.total > 0 && !aligned16(workspace))) {
    set_error("fused moe: workspace too small or misaligned (%lld < %lld bytes)",
              (long long)workspace_bytes, (long long)p.total);
    return MXFP4_ERR_VALUE;
  }
  if (routes == 0) return MXFP4_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Few routes on the W4A16 path: the decode kernels find each route's rows
  // from the top-k ids (direct routing, as in the MoE layer), so no routing
  // launch; a route whose id is outside [0, E) writes zeros to its row.
  const SoftPath path = soft_path(a_dtype, c_dtype, pre_b != nullptr);
  const int64_t lim = (int64_t)1 << 31;
  if ((path == SOFT_W4A16 || path == SOFT_W4A16_PRE) && routes <= kDirectRoutes &&
      n * (k / 2) < lim && a_rows * a_row_stride * elem_size(a_dtype) < lim) {
    GemmArgs g = routed_args(a, a_rows, a_row_stride, a_mx, b, b_mx, num_experts, n, k, c, n,
                             a_scale, b_scale, topk_weights, mul_routed_weight, nullptr, nullptr,
                             nullptr, routes, 16, routes, top_k);
    g.route_ids = topk_ids;
    g.ids64 = ids_dtype == MXFP4_DT_I64;
    g.zero_dropped = 1;
    return dispatch_gemm(g, a_dtype, c_dtype, EPI_STORE, st);
  }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + p.off_counts);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + p.off_sorted);
  int32_t* experts = reinterpret_cast<int32_t*>(ws + p.off_experts);
  int32_t* npp = reinterpret_cast<int32_t*>(ws + p.off_npp);
  if (p.zero_c) {
    const int64_t bytes = routes * n * elem_size(c_dtype);
    const int64_t blocks = std::min<int64_t>((bytes / 16 + 255) / 256 + 1, 4096);
    zero_fill<<<(unsigned)blocks, 256, 0, st>>>(static_cast<uint8_t*>(c), bytes);
    rc = launch_status("fused moe zero fill launch");
    if (rc) return rc;
  }
  rc = do_align(topk_ids, ids_dtype, routes, p.align_experts, p.block_m, sorted, experts, npp,
                counts, p.nchunks, st, p.drop_to);
  if (rc) return rc;
  GemmArgs g = routed_args(a, a_rows, a_row_stride, a_mx, b, b_mx, num_experts, n, k, c, n,
                           a_scale, b_scale, topk_weights, mul_routed_weight, sorted, experts, npp,
                           p.max_sorted, p.block_m, routes, top_k);
  set_prepacked(g, pre_b, pre_s, n, k);
  return dispatch_gemm(g, a_dtype, c_dtype, EPI_STORE, st);
}

extern "C" int mxfp4_linear_w4a16_workspace_size(int64_t m, int64_t k, int64_t n, int64_t* bytes) {
  if (bytes == nullptr || m < 0 || k <= 0 || n <= 0) {
    set_error("linear workspace size: invalid arguments");
    return MXFP4_ERR_VALUE;
  }
  *bytes = (m > 0 && k % 128 == 0) ? splitk_ws_bytes(m, k, n) : 0;
  return MXFP4_OK;
}

extern "C" int mxfp4_linear_w4a16(const void* x, int x_dtype, int64_t m, int64_t k,
                                  int64_t x_row_stride, const uint8_t* packed,
                                  const uint8_t* scales, int64_t n, const void* bias, void* out,
                                  void* stream) {
  return mxfp4_linear_w4a16_ws(x, x_dtype, m, k, x_row_stride, packed, scales, n, bias, out,
                               nullptr, 0, stream);
}

extern "C" int mxfp4_linear_w4a16_ws(const void* x, int x_dtype, int64_t m, int64_t k,
                                     int64_t x_row_stride, const uint8_t* packed,
                                     const uint8_t* scales, int64_t n, const void* bias, void* out,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  return mxfp4_linear_w4a16_pre(x, x_dtype, m, k, x_row_stride, packed, scales, nullptr, nullptr,
                                n, bias, out, workspace, workspace_bytes, stream);
}

extern "C" int mxfp4_linear_w4a16_pre(const void* x, int x_dtype, int64_t m, int64_t k,
                                      int64_t x_row_stride, const uint8_t* packed,
                                      const uint8_t* scales, const uint8_t* pre_b,
                                      const uint16_t* pre_s, int64_t n, const void* bias, void* out,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
  if (x_dtype != MXFP4_DT_BF16 && x_dtype != MXFP4_DT_F16) {
    set_error("x must be fp16 or bf16, got dtype %d", x_dtype);
    return MXFP4_ERR_TYPE;
  }
  if (k <= 0 || k % 128 != 0) {
    set_error("logical K must be divisible by 128, got %lld", (long long)k);
    return MXFP4_ERR_VALUE;
  }
  if (n <= 0 || n > 0x7FFFFFFF || k > 0x7FFFFFFF || m < 0) {
    set_error("linear: invalid sizes");
    return MXFP4_ERR_VALUE;
  }
  if (!aligned16(x) || !aligned16(packed) || (x_row_stride * 2) % 16 || x_row_stride < k) {
    set_error("linear: activation/weight rows must be 16-byte aligned");
    return MXFP4_ERR_VALUE;
  }
  if (m == 0) return MXFP4_OK;
  GemmArgs g = {};
  g.a = x;
  g.a_rows = m;
  g.lda = x_row_stride;
  g.b = packed;
  g.bs = scales;
  g.b_n = k / 2;
  g.bs_n = k / 32;
  g.c = out;
  g.ldc = n;
  g.bias = bias;
  g.m = m;
  g.num_valid = m;
  g.n = (int32_t)n;
  g.k = (int32_t)k;
  g.top_k = 1;
  g.block_m = 16;
  if ((pre_b == nullptr) != (pre_s == nullptr)) {
    set_error("linear: the prepacked nibbles and scales come together");
    return MXFP4_ERR_VALUE;
  }
  g.pre_b = pre_b;
  g.pre_s = pre_s;
  if (workspace != nullptr) {
    const int64_t need = splitk_ws_bytes(m, k, n);
    if (need > 0 && (workspace_bytes < need || !aligned16(workspace))) {
      set_error("linear: workspace must be 16-byte aligned and hold %lld bytes", (long long)need);
      return MXFP4_ERR_VALUE;
    }
    if (need > 0) g.splitk_ws = static_cast<float*>(workspace);
  }
  return launch_w4a16(g, x_dtype, EPI_STORE, static_cast<hipStream_t>(stream));
}

extern "C" int mxfp4_linear_w4a4(const uint8_t* a, const uint8_t* a_mx, int64_t m, int64_t k,
                                 const uint8_t* b, const uint8_t* b_mx, int64_t n, void* out,
                                 int out_dtype, void* stream) {
  if (out_dtype != MXFP4_DT_BF16 && out_dtype != MXFP4_DT_F16 && out_dtype != MXFP4_DT_F32) {
    set_error("w4a4: unsupported output dtype %d", out_dtype);
    return MXFP4_ERR_TYPE;
  }
  if (k <= 0 || k % 32 != 0 || n <= 0 || m < 0 || n > 0x7FFFFFFF || k > 0x7FFFFFFF) {
    set_error("logical K must be divisible by 32, got %lld", (long long)k);
    return MXFP4_ERR_VALUE;
  }
  if (!aligned16(a) || !aligned16(b)) {
    set_error("w4a4: packed rows must be 16-byte aligned");
    return MXFP4_ERR_VALUE;
  }
  if (m == 0) return MXFP4_OK;
  GemmArgs g = {};
  g.a = a;
  g.a_mx = a_mx;
  g.a_rows = m;
  g.lda = k / 2;
  g.lda_mx = k / 32;
  g.b = b;
  g.bs = b_mx;
  g.b_n = k / 2;
  g.bs_n = k / 32;
  g.c = out;
  g.ldc = n;
  g.m = m;
  g.num_valid = m;
  g.n = (int32_t)n;
  g.k = (int32_t)k;
  g.top_k = 1;
  g.block_m = 16;
  return launch_w4a4(g, out_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int mxfp4_moe_layer_workspace_size(int64_t m, int top_k, int num_experts,
                                              int64_t hidden, int64_t inter, int64_t* bytes) {
  if (m < 0 || top_k < 1 || num_experts < 1 || num_experts > kMaxExperts || hidden <= 0 ||
      inter <= 0) {
    set_error("moe layer: invalid sizes");
    return MXFP4_ERR_VALUE;
  }
  // either weight layout's plan fits (the caller may pass prepacked copies)
  const int64_t a = plan_layer(m, top_k, num_experts, hidden, inter, 2, true).total;
  const int64_t b = plan_layer(m, top_k, num_experts, hidden, inter, 2, false).total;
  *bytes = a > b ? a : b;
  return MXFP4_OK;
}

extern "C" int mxfp4_moe_layer(const void* x, int x_dtype, int64_t m, int64_t hidden,
                               const uint8_t* w13, const uint8_t* s13, const uint8_t* w2,
                               const uint8_t* s2, int num_experts, int64_t inter,
                               const float* topk_weights, const void* topk_ids, int ids_dtype,
                               int top_k, void* out, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  return mxfp4_moe_layer_pre(x, x_dtype, m, hidden, w13, s13, nullptr, nullptr, w2, s2, nullptr,
                             nullptr, num_experts, inter, topk_weights, topk_ids, ids_dtype, top_k,
                             out, workspace, workspace_bytes, stream);
}

extern "C" int mxfp4_moe_layer_pre(const void* x, int x_dtype, int64_t m, int64_t hidden,
                                   const uint8_t* w13, const uint8_t* s13, const uint8_t* pre13_b,
                                   const uint16_t* pre13_s, const uint8_t* w2, const uint8_t* s2,
                                   const uint8_t* pre2_b, const uint16_t* pre2_s, int num_experts,
                                   int64_t inter, const float* topk_weights, const void* topk_ids,
                                   int ids_dtype, int top_k, void* out, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  if ((pre13_b == nullptr) != (pre13_s == nullptr) || (pre2_b == nullptr) != (pre2_s == nullptr)) {
    set_error("moe layer: the prepacked nibbles and scales come together");
    return MXFP4_ERR_VALUE;
  }
  if (x_dtype != MXFP4_DT_BF16 && x_dtype != MXFP4_DT_F16) {
    set_error("moe layer: x must be fp16 or bf16");
    return MXFP4_ERR_TYPE;
  }
  if (hidden % 32 || inter % 32 || hidden <= 0 || inter <= 0 || hidden > 0x3FFFFFFF ||
      inter > 0x3FFFFFFF) {
    set_error("moe layer: hidden and intermediate sizes must be multiples of 32");
    return MXFP4_ERR_VALUE;
  }
  int rc = check_align_args(m * top_k, num_experts, 16, ids_dtype);
  if (rc) return rc;
  if (!aligned16(x) || !aligned16(w13) || !aligned16(w2) || !aligned16(out) ||
      !aligned16(workspace)) {
    set_error("moe layer: buffers must be 16-byte aligned");
    return MXFP4_ERR_VALUE;
  }
  const LayerPlan p = plan_layer(m, top_k, num_experts, hidden, inter, 2, pre13_b != nullptr);
  if (workspace_bytes < p.total) {
    set_error("moe layer: workspace too small (%lld < %lld)", (long long)workspace_bytes,
              (long long)p.total);
    return MXFP4_ERR_VALUE;
  }
  if (m == 0) return MXFP4_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + p.off_counts);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + p.off_sorted);
  int32_t* experts = reinterpret_cast<int32_t*>(ws + p.off_experts);
  int32_t* npp = reinterpret_cast<int32_t*>(ws + p.off_npp);
  void* h = ws + p.off_h;
  void* d = ws + p.off_d;

  // Few routes: the GEMMs find their rows from the top-k ids directly
  // (direct routing), so no routing metadata is built.
  const bool direct = p.routes <= kDirectRoutes && inter * hidden < ((int64_t)1 << 31);
  if (!direct) {
    rc = do_align(topk_ids, ids_dtype, p.routes, num_experts, p.block_m, sorted, experts, npp,
                  counts, p.nchunks, st);
    if (rc) return rc;
  }

  // gate_up with the fused SiLU*mul epilogue: h[r, :inter]
  GemmArgs g = {};
  g.a = x;
  g.a_rows = m;
  g.lda = hidden;
  g.b = w13;
  g.bs = s13;
  g.b_n = hidden / 2;
  g.b_e = 2 * inter * (hidden / 2);
  g.bs_n = hidden / 32;
  g.bs_e = 2 * inter * (hidden / 32);
  g.c = h;
  g.ldc = inter;
  g.sorted_ids = sorted;
  g.expert_ids = experts;
  g.num_post_padded = npp;
  g.m = p.max_sorted;
  g.num_valid = p.routes;
  g.n = (int32_t)inter;
  g.k = (int32_t)hidden;
  g.top_k = top_k;
  g.block_m = p.block_m;
  g.inter = (int32_t)inter;
  g.num_experts = num_experts;
  g.pre_b = pre13_b;
  g.pre_s = pre13_s;
  g.pre_b_e = prepacked_nibble_bytes(2 * inter, hidden);
  g.pre_s_e = prepacked_scale_bytes(2 * inter, hidden);
  if (direct) {
    g.sorted_ids = nullptr;
    g.expert_ids = nullptr;
    g.num_post_padded = nullptr;
    g.route_ids = topk_ids;
    g.ids64 = ids_dtype == MXFP4_DT_I64;
  }
  rc = launch_w4a16(g, x_dtype, EPI_SILU_MUL, st);
  if (rc) return rc;
  if (direct && top_k <= 16) {
    // down with the route weight and the top-k sum in one kernel
    return launch_moe_down_topk(h, w2, s2, topk_weights, topk_ids, ids_dtype == MXFP4_DT_I64, m,
                                top_k, hidden, inter, num_experts, out, x_dtype, st);
  }

  // down with the route weight: d[r, :hidden]
  GemmArgs g2 = g;
  g2.a = h;
  g2.a_rows = p.routes;
  g2.lda = inter;
  g2.b = w2;
  g2.bs = s2;
  g2.b_n = inter / 2;
  g2.b_e = hidden * (inter / 2);
  g2.bs_n = inter / 32;
  g2.bs_e = hidden * (inter / 32);
  g2.c = d;
  g2.ldc = hidden;
  g2.route_w = topk_weights;
  g2.n = (int32_t)hidden;
  g2.k = (int32_t)inter;
  g2.top_k = 1;
  g2.inter = 0;
  g2.pre_b = pre2_b;
  g2.pre_s = pre2_s;
  g2.pre_b_e = prepacked_nibble_bytes(hidden, inter);
  g2.pre_s_e = prepacked_scale_bytes(hidden, inter);
  rc = launch_w4a16(g2, x_dtype, EPI_STORE, st);
  if (rc) return rc;

  // top-k combine
  const int64_t total = m * (hidden / 8);
  const int grid = (int)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  if (x_dtype == MXFP4_DT_BF16) {
    if (ids_dtype == MXFP4_DT_I32)
      topk_sum<__bf16, int32_t><<<grid, 256, 0, st>>>(static_cast<const __bf16*>(d),
                                                      static_cast<const int32_t*>(topk_ids), m,
                                                      top_k, hidden, num_experts,
                                                      static_cast<__bf16*>(out));
    else
      topk_sum<__bf16, int64_t><<<grid, 256, 0, st>>>(static_cast<const __bf16*>(d),
                                                      static_cast<const int64_t*>(topk_ids), m,
                                                      top_k, hidden, num_experts,
                                                      static_cast<__bf16*>(out));
  } else {
    if (ids_dtype == MXFP4_DT_I32)
      topk_sum<_Float16, int32_t><<<grid, 256, 0, st>>>(static_cast<const _Float16*>(d),
                                                        static_cast<const int32_t*>(topk_ids), m,
                                                        top_k, hidden, num_experts,
                                                        static_cast<_Float16*>(out));
    else
      topk_sum<_Float16, int64_t><<<grid, 256, 0, st>>>(static_cast<const _Float16*>(d),
                                                        static_cast<const int64_t*>(topk_ids), m,
                                                        top_k, hidden, num_experts,
                                                        static_cast<_Float16*>(out));
  }
  return launch_status("moe topk sum launch");
}

// ---------------------------------------------------------------- allocation-free layer
// mxfp4_moe_layer for callers that cannot allocate device memory (code under
// HIP graph capture, serving loops, harnesses that forbid hipMalloc): the
// layer's workspace -- routing metadata and the h / d intermediates -- is a
// file-scope device array of kNoAllocScratchBytes, which every GPU the
// library runs on holds until the process ends.  The host side never uses
// the array's name as an address: its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) and kept here.
// No kernel of the layer needs its workspace cleared: every word a kernel
// reads was written earlier in the same call (the routing counts per chunk,
// h and d for every route the later kernels read).  Calls that overlap on
// one GPU share the array and race.

namespace {

constexpr int64_t kNoAllocScratchBytes = MXFP4_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device); nullptr with the error set on failure.
void* scratch_on_current_device() {
  int dev = -1;
  if (hip_status(hipGetDevice(&dev), "hipGetDevice") != MXFP4_OK) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("moe layer (no-alloc): device %d out of range", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)") !=
        MXFP4_OK)
      return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int mxfp4_moe_layer_noalloc(const void* x, int x_dtype, int64_t m, int64_t hidden,
                                       const uint8_t* w13, const uint8_t* s13, const uint8_t* w2,
                                       const uint8_t* s2, int num_experts, int64_t inter,
                                       const float* topk_weights, const void* topk_ids,
                                       int ids_dtype, int top_k, void* out, void* stream) {
  int64_t need = 0;
  int rc = mxfp4_moe_layer_workspace_size(m, top_k, num_experts, hidden, inter, &need);
  if (rc) return rc;
  if (need > kNoAllocScratchBytes) {
    set_error("moe layer (no-alloc): %lld tokens x top-%d need a %lld-byte workspace, above the "
              "%lld bytes of the fixed scratch; use mxfp4_moe_layer with a workspace",
              (long long)m, top_k, (long long)need, (long long)kNoAllocScratchBytes);
    return MXFP4_ERR_VALUE;
  }
  void* ws = scratch_on_current_device();
  if (ws == nullptr) return MXFP4_ERR_HIP;
  return mxfp4_moe_layer(x, x_dtype, m, hidden, w13, s13, w2, s2, num_experts, inter,
                         topk_weights, topk_ids, ids_dtype, top_k, out, ws, kNoAllocScratchBytes,
                         stream);
}
