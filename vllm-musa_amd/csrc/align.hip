// moe_align_block_size: group routes by expert, pad each expert's segment to
// a multiple of the block size, and keep ascending route order inside each
// segment (a stable counting sort), so the result is deterministic.
//
// Each 1024-thread workgroup places one contiguous chunk of 1024 routes (more
// per workgroup only beyond 256 workgroups):
//   1. LDS histogram of all the (mapped) expert ids, and of those before the
//      chunk (every workgroup reads all ids: no global scratch and no second
//      launch, at numel * 4 bytes of L2 reads per workgroup);
//   2. block-wide exclusive scan of the padded counts -> segment bases;
//   3. stable placement of the chunk, 1024 routes per step: the rank of a
//      route among the same-expert routes of its wave comes from bit-sliced
//      ballots (one 64-bit ballot per expert-id bit, no loops over lanes), the
//      rank across the 16 waves of the step from a [wave][expert] count table
//      in LDS, and the rank across steps and earlier chunks from a running
//      per-expert counter that starts at the count before the chunk.
// With a counts buffer (the bf16 layers' workspace, align_routes) step 1
// runs as its own launch instead: each workgroup histograms only its chunk into
// counts[blk][E] (PHASE 1), and the placement launch (PHASE 2) sums the
// chunk histograms, all of them and those before its chunk.  Adds to LDS
// run at about one route per clock per CU, so histogramming all routes in
// every workgroup (PHASE 0) costs numel clocks: 29 us at 65536 routes.
// Workgroup 0 also writes the per-call outputs (num_tokens_post_pad, offsets,
// active experts, expert_ids).  The sentinel `numel` goes to every position
// of sorted_token_ids that no route takes, exactly once, so no ordering
// between writers is needed: expert e's padding by one wave of workgroup
// e % nblk (64 consecutive positions per store), the unused tail by all
// workgroups in turn.
#include "quant_dev.h"

namespace vmamd {

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / kWave;  // 16
constexpr int kMaxAlignExperts = 1024;

__device__ __forceinline__ int mapped_expert(const int32_t* __restrict__ ids, int64_t r, int E,
                                             const int32_t* __restrict__ map, int64_t map_len) {
  int e = ids[r];
  if (map) {
    if (e < 0 || e >= map_len) return -1;
    e = map[e];
  }
  return (e >= 0 && e < E) ? e : -1;
}

// Routes placed per workgroup: one placement step (several steps per
// workgroup only beyond 256 workgroups).
constexpr int64_t kAlignChunk = kAlignThreads;

template <int PHASE>
__device__ __forceinline__ void align_body(
    int blk, int nblk, const int32_t* __restrict__ ids, int64_t numel, int64_t chunk, int E, int bs,
    const int32_t* __restrict__ map, int64_t map_len, int32_t* __restrict__ sorted, int64_t capacity,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp, int32_t* __restrict__ offsets_out,
    int32_t* __restrict__ scatter_idx, int32_t* __restrict__ active_out,
    int32_t* __restrict__ num_active_out, int32_t* __restrict__ counts) {
  __shared__ int cnt[kMaxAlignExperts];
  __shared__ int base[kMaxAlignExperts + 1];
  __shared__ int run[kMaxAlignExperts];
  __shared__ uint16_t wcnt[kAlignWaves][kMaxAlignExperts];
  __shared__ int wave_tot[kAlignWaves];

  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;

  for (int e = tid; e < E; e += kAlignThreads) {
    cnt[e] = 0;
    run[e] = 0;
  }
  __syncthreads();

  // 1. histograms of the routes before this chunk (run) and of the others
  // (cnt, then cnt += run: all routes), one LDS add per route; each thread
  // has 8 ids in flight (one per strided slot) before its adds.
  const int64_t c_begin = static_cast<int64_t>(blk) * chunk;
  const int64_t c_end = min(numel, c_begin + chunk);
  if constexpr (PHASE == 1) {  // this chunk's histogram only
    for (int64_t r = c_begin + tid; r < c_end; r += kAlignThreads) {
      const int e = mapped_expert(ids, r, E, map, map_len);
      if (e >= 0) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    for (int e = tid; e < E; e += kAlignThreads) counts[static_cast<int64_t>(blk) * E + e] = cnt[e];
    return;
  }
  constexpr int kHistU = 8;
  if constexpr (PHASE == 2) {  // the chunk histograms: all (cnt) and before this chunk (run)
    for (int e = tid; e < E; e += kAlignThreads) {
      int all = 0, before = 0;
      for (int b0 = 0; b0 < nblk; b0 += kHistU) {
        int v[kHistU];
#pragma unroll
        for (int u = 0; u < kHistU; ++u) v[u] = b0 + u < nblk ? counts[static_cast<int64_t>(b0 + u) * E + e] : 0;
#pragma unroll
        for (int u = 0; u < kHistU; ++u) {
          all += v[u];
          before += b0 + u < blk ? v[u] : 0;
        }
      }
      cnt[e] = all;
      run[e] = before;
    }
  }
  for (int64_t r0 = tid; PHASE == 0 && r0 < numel; r0 += kHistU * kAlignThreads) {
    int ev[kHistU];
#pragma unroll
    for (int u = 0; u < kHistU; ++u) {
      const int64_t r = r0 + u * kAlignThreads;
      ev[u] = r < numel ? mapped_expert(ids, r, E, map, map_len) : -1;
    }
#pragma unroll
    for (int u = 0; u < kHistU; ++u)
      if (ev[u] >= 0) atomicAdd(r0 + u * kAlignThreads < c_begin ? &run[ev[u]] : &cnt[ev[u]], 1);
  }
  __syncthreads();
  if constexpr (PHASE == 0)
    for (int e = tid; e < E; e += kAlignThreads) cnt[e] += run[e];
  __syncthreads();
  const bool lead = blk == 0;  // writes the per-call outputs

  // 2. exclusive scan of padded counts (E <= 1024: one expert per thread)
  int padded = 0;
  if (tid < E) padded = (cnt[tid] + bs - 1) / bs * bs;
  int incl = padded;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += o;
  }
  if (lane == kWave - 1) wave_tot[wave] = incl;
  __syncthreads();
  int wave_off = 0;
  for (int w = 0; w < wave; ++w) wave_off += wave_tot[w];
  if (tid < E) base[tid] = wave_off + incl - padded;
  if (tid == kAlignThreads - 1) base[E] = wave_off + incl;  // last thread sees the total
  __syncthreads();
  const int total = base[E];
  if (lead && tid == 0) ntpp[0] = total;
  if (lead && offsets_out)
    for (int e = tid; e <= E; e += kAlignThreads) offsets_out[e] = base[e];

  // compact list of the experts that received routes (ascending ids)
  if (lead && active_out) {
    const bool act = tid < E && cnt[tid] > 0;
    const uint64_t m = ballot(act);
    const int below = __popcll(m & ((lane == 0) ? 0ull : (~0ull >> (kWave - lane))));
    __syncthreads();  // wave_tot is reused below
    if (lane == 0) wave_tot[wave] = __popcll(m);
    __syncthreads();
    int off = 0;
    for (int w = 0; w < wave; ++w) off += wave_tot[w];
    if (act) active_out[off + below] = tid;
    if (tid == kAlignThreads - 1) num_active_out[0] = off + __popcll(m);
    __syncthreads();
  }

  // expert_ids: binary search of the segment holding each block
  const int64_t nblocks = lead ? (capacity + bs - 1) / bs : 0;
  for (int64_t b = tid; b < nblocks; b += kAlignThreads) {
    int out = -1;
    const int64_t pos = b * bs;
    if (pos < total) {
      int lo = 0, hi = E - 1;  // largest e with base[e] <= pos
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (base[mid] <= pos) lo = mid; else hi = mid - 1;
      }
      out = lo;
    }
    expert_ids[b] = out;
  }
  // sentinel for the padding of each segment and the unused tail
  const int32_t sentinel = static_cast<int32_t>(numel);
  for (int e = blk + nblk * wave; e < E; e += nblk * kAlignWaves)
    for (int p = base[e] + cnt[e] + lane; p < base[e + 1]; p += kWave) sorted[p] = sentinel;
  for (int64_t p = total + static_cast<int64_t>(blk) * kAlignThreads + tid; p < capacity;
       p += static_cast<int64_t>(nblk) * kAlignThreads)
    sorted[p] = sentinel;

  // 3. stable placement
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  for (int64_t c0 = c_begin; c0 < c_end; c0 += kAlignThreads) {
    for (int i = tid; i < kAlignWaves * E; i += kAlignThreads) wcnt[i / E][i % E] = 0;
    const int64_t r = c0 + tid;
    const int e = r < c_end ? mapped_expert(ids, r, E, map, map_len) : -1;
    const bool valid = e >= 0;
    uint64_t same = ballot(valid);
#pragma unroll 1
    for (int b = 0; b < nbits; ++b) {
      const uint64_t on = ballot(valid && ((e >> b) & 1));
      same &= ((e >> b) & 1) ? on : ~on;
    }
    __syncthreads();
    const int rank_in_wave = __popcll(same & lt_mask);
    if (valid && rank_in_wave == 0) wcnt[wave][e] = static_cast<uint16_t>(__popcll(same));
    __syncthreads();
    if (valid) {
      int before = run[e];
      for (int w = 0; w < wave; ++w) before += wcnt[w][e];
      const int pos = base[e] + before + rank_in_wave;
      if (pos < base[e + 1]) {  // always true; keeps a corrupted count from writing out of range
        sorted[pos] = static_cast<int32_t>(r);
        if (scatter_idx) scatter_idx[r] = pos;
      }
    } else if (r < c_end && scatter_idx) {
      scatter_idx[r] = -1;
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += kAlignThreads) {
      int add = 0;
      for (int w = 0; w < kAlignWaves; ++w) add += wcnt[w][ee];
      run[ee] += add;
    }
    __syncthreads();
  }
}


template <int PHASE>
__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int64_t chunk, int E, int bs,
    const int32_t* __restrict__ map, int64_t map_len, int32_t* __restrict__ sorted, int64_t capacity,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp, int32_t* __restrict__ offsets_out,
    int32_t* __restrict__ scatter_idx, int32_t* __restrict__ active_out,
    int32_t* __restrict__ num_active_out, int32_t* __restrict__ counts) {
  align_body<PHASE>(blockIdx.x, gridDim.x, ids, numel, chunk, E, bs, map, map_len, sorted, capacity,
                    expert_ids, ntpp, offsets_out, scatter_idx, active_out, num_active_out, counts);
}

// The MoE layer's two independent first steps in one launch: workgroups
// [0, align_groups) run moe_align_block_size, the others the 1x128 fp8
// quantiser of the bf16 activations (kAlignThreads / 16 groups each).  The
// alignment keeps its one-launch form here: its all-route histogram runs
// beside the quantiser's workgroups (measured at T=4096: one launch 34.0 us,
// histograms + quantiser then placement 27.3 + 9.8 us).
__global__ __launch_bounds__(kAlignThreads) void moe_align_quant_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int64_t chunk, int align_groups, int E, int bs,
    const int32_t* __restrict__ map, int64_t map_len, int32_t* __restrict__ sorted, int64_t capacity,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp, int32_t* __restrict__ offsets_out,
    int32_t* __restrict__ active_out, int32_t* __restrict__ num_active_out,
    const uint16_t* __restrict__ x, int64_t groups_per_row, int64_t num_groups, bool vec,
    uint8_t* __restrict__ xq, float* __restrict__ xs) {
  if (static_cast<int>(blockIdx.x) < align_groups) {
    align_body<0>(blockIdx.x, align_groups, ids, numel, chunk, E, bs, map, map_len, sorted, capacity,
                  expert_ids, ntpp, offsets_out, nullptr, active_out, num_active_out, nullptr);
    return;
  }
  constexpr int kGroupsPerAlignBlock = kAlignThreads / kLanesPerGroup;
  const int64_t g = static_cast<int64_t>(blockIdx.x - align_groups) * kGroupsPerAlignBlock +
                    threadIdx.x / kLanesPerGroup;
  if (g >= num_groups) return;
  const int64_t cols = groups_per_row * kGroup;
  group_quant_group<kBF16>(x, cols, groups_per_row, g, threadIdx.x % kLanesPerGroup, vec, 1e-10f,
                           -448.f, 448.f, xq, cols, xs, groups_per_row, 1);
}

// As moe_align_quant_kernel, with the w4afp8 per-row quantiser (w4 order and
// block corrections; one launch measured 26.2 us at T=4096 against 22.1 + 8.6
// for histograms + quantiser then placement).  CPL > 0: a quant workgroup quantises one row per wave
// (cols <= 512 * CPL); CPL = 0: kAlignThreads / kRowThreads rows, one per
// 256-thread part.
// One thread per row of a W4ScalesT matrix (row n of expert e: kp words in,
// word p to out[e][p][n]): the row read 8 bytes at a time, each word
// written where the threads of neighbouring rows write its neighbours.
__device__ __forceinline__ void w4_scales_t_rows(const W4ScalesT& t, int64_t g) {
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int64_t nrow = static_cast<int64_t>(t.E) * t.n[m];
    if (t.in[m] && g < nrow) {
      const int kp = t.kp[m], n = t.n[m];
      const int64_t e = g / n, r = g - e * n;
      const uint2* src = reinterpret_cast<const uint2*>(t.in[m] + g * kp);
      uint32_t* dst = t.out[m] + e * kp * n + r;
      for (int p = 0; p < kp; p += 2) {
        const uint2 v = src[p / 2];
        dst[static_cast<int64_t>(p) * n] = v.x;
        dst[static_cast<int64_t>(p + 1) * n] = v.y;
      }
      return;
    }
    if (t.in[m]) g -= nrow;
  }
}

template <int CPL>
__global__ __launch_bounds__(kAlignThreads) void moe_align_rowquant_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int64_t chunk, int align_groups, int E, int bs,
    const int32_t* __restrict__ map, int64_t map_len, int32_t* __restrict__ sorted, int64_t capacity,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp, int32_t* __restrict__ offsets_out,
    int32_t* __restrict__ active_out, int32_t* __restrict__ num_active_out,
    const uint16_t* __restrict__ x, int64_t rows, int cols, uint8_t* __restrict__ xq,
    float* __restrict__ xs, float* __restrict__ xcorr, int quant_groups, W4ScalesT sct) {
  if (static_cast<int>(blockIdx.x) < align_groups) {
    align_body<0>(blockIdx.x, align_groups, ids, numel, chunk, E, bs, map, map_len, sorted, capacity,
                  expert_ids, ntpp, offsets_out, nullptr, active_out, num_active_out, nullptr);
    return;
  }
  if (static_cast<int>(blockIdx.x) >= align_groups + quant_groups) {  // the scale transpositions
    w4_scales_t_rows(sct, static_cast<int64_t>(blockIdx.x - align_groups - quant_groups) * kAlignThreads +
                              threadIdx.x);
    return;
  }
  if constexpr (CPL > 0) {
    const int64_t row = static_cast<int64_t>(blockIdx.x - align_groups) * (kAlignThreads / kWave) +
                        threadIdx.x / kWave;
    row_quant_wave<true, CPL>(x, cols, cols, 1e-4f, -448.f, 448.f, xq, xs, row, row < rows, xcorr);
  } else {
    constexpr int kParts = kAlignThreads / kRowThreads;
    __shared__ float red[kAlignThreads / kWave];
    const int part = threadIdx.x / kRowThreads;
    const int64_t row = static_cast<int64_t>(blockIdx.x - align_groups) * kParts + part;
    row_quant_part<true>(x, cols, cols, 1e-4f, -448.f, 448.f, xq, xs, row, row < rows,
                         threadIdx.x % kRowThreads, red + part * (kRowThreads / kWave), xcorr);
  }
}

}  // namespace vmamd

using namespace vmamd;

namespace vmamd {
// Work split of moe_align_block_size: one workgroup per chunk of 1024 routes,
// at most 256 workgroups.
static void align_grid(int64_t numel, int64_t& chunk, int& groups) {
  chunk = kAlignChunk * std::max<int64_t>(1, (numel + kAlignChunk * 256 - 1) / (kAlignChunk * 256));
  groups = static_cast<int>((numel + chunk - 1) / chunk);
}

size_t align_counts_bytes(int64_t numel, int E) {
  int64_t chunk;
  int groups;
  align_grid(numel, chunk, groups);
  return static_cast<size_t>(std::max(groups, 1)) * E * 4;
}

// The placement launch after a PHASE 1 histogram launch.
static void align_place(const int32_t* ids, int64_t numel, int64_t chunk, int groups, int E, int bs,
                        const int32_t* map, int64_t map_len, int32_t* sorted, int64_t capacity, int32_t* expert_ids,
                        int32_t* ntpp, int32_t* offsets, int32_t* active, int32_t* num_active, int32_t* counts,
                        hipStream_t st) {
  moe_align_kernel<2><<<groups, kAlignThreads, 0, st>>>(ids, numel, chunk, E, bs, map, map_len, sorted, capacity,
                                                        expert_ids, ntpp, offsets, nullptr, active, num_active,
                                                        counts);
}

int align_routes(const int32_t* topk_ids, int64_t numel, int num_experts, int block_size,
                 const int32_t* expert_map, int64_t expert_map_len, int32_t* sorted, int64_t capacity,
                 int32_t* expert_ids, int32_t* ntpp, int32_t* offsets, int32_t* active, int32_t* num_active,
                 int32_t* counts, hipStream_t st) {
  int64_t chunk;
  int groups;
  align_grid(numel, chunk, groups);
  if (counts == nullptr || groups <= 1)
    return vmamd_moe_align_block_size(topk_ids, numel, num_experts, block_size, expert_map, expert_map_len, sorted,
                                      capacity, expert_ids, ntpp, offsets, nullptr, active, num_active,
                                      reinterpret_cast<vmamd_stream_t>(st));
  moe_align_kernel<1><<<groups, kAlignThreads, 0, st>>>(topk_ids, numel, chunk, num_experts, block_size, expert_map,
                                                        expert_map_len, sorted, capacity, expert_ids, ntpp, offsets,
                                                        nullptr, active, num_active, counts);
  int rc = check_launch("moe align (histograms)");
  if (rc) return rc;
  align_place(topk_ids, numel, chunk, groups, num_experts, block_size, expert_map, expert_map_len, sorted, capacity,
              expert_ids, ntpp, offsets, active, num_active, counts, st);
  return check_launch("moe align (placement)");
}

int align_and_group_quant_fp8(const int32_t* topk_ids, int64_t numel, int num_experts,
                              int block_size, const int32_t* expert_map, int64_t expert_map_len,
                              int32_t* sorted, int64_t capacity, int32_t* expert_ids, int32_t* ntpp,
                              int32_t* offsets, int32_t* active, int32_t* num_active,
                              const void* x, int64_t rows, int64_t cols, uint8_t* xq, float* xs,
                              hipStream_t st) {
  const char* who = "moe align + quant";
  VMAMD_REQUIRE(num_experts > 0 && num_experts <= kMaxAlignExperts && block_size > 0, "%s: bad sizes",
                who);
  VMAMD_REQUIRE(numel >= 0 && numel < (1ll << 31) - 1 && capacity < (1ll << 31) &&
                    capacity >= numel + static_cast<int64_t>(num_experts) * (block_size - 1),
                "%s: bad route count or capacity", who);
  VMAMD_REQUIRE(!expert_map || expert_map_len > 0, "%s: empty expert_map", who);
  VMAMD_REQUIRE(rows >= 0 && cols > 0 && cols % kGroup == 0, "%s: cols must be a multiple of 128", who);
  VMAMD_REQUIRE((topk_ids || numel == 0) && sorted && expert_ids && ntpp && (x || rows == 0) &&
                    (reinterpret_cast<uintptr_t>(xq) & 7) == 0,
                "%s: null or misaligned pointer", who);
  int64_t chunk;
  int groups;
  align_grid(numel, chunk, groups);
  groups = std::max(groups, 1);
  const int64_t groups_per_row = cols / kGroup;
  const int64_t num_groups = rows * groups_per_row;
  const int64_t qblocks = (num_groups + kAlignThreads / kLanesPerGroup - 1) / (kAlignThreads / kLanesPerGroup);
  const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0;  // rows of cols % 128 == 0 bf16 stay aligned
  moe_align_quant_kernel<<<static_cast<int>(groups + qblocks), kAlignThreads, 0, st>>>(
      topk_ids, numel, chunk, groups, num_experts, block_size, expert_map, expert_map_len, sorted,
      capacity, expert_ids, ntpp, offsets, active, num_active, static_cast<const uint16_t*>(x),
      groups_per_row, num_groups, vec, xq, xs);
  return check_launch(who);
}
int align_and_row_quant_fp8(const int32_t* topk_ids, int64_t numel, int num_experts,
                            int block_size, const int32_t* expert_map, int64_t expert_map_len,
                            int32_t* sorted, int64_t capacity, int32_t* expert_ids, int32_t* ntpp,
                            int32_t* offsets, int32_t* active, int32_t* num_active, const void* x,
                            int64_t rows, int64_t cols, uint8_t* xq, float* xs, float* xcorr,
                            hipStream_t st, const W4ScalesT* sct) {
  const char* who = "moe align + row quant";
  VMAMD_REQUIRE(num_experts > 0 && num_experts <= kMaxAlignExperts && block_size > 0, "%s: bad sizes",
                who);
  VMAMD_REQUIRE(numel >= 0 && numel < (1ll << 31) - 1 && capacity < (1ll << 31) &&
                    capacity >= numel + static_cast<int64_t>(num_experts) * (block_size - 1),
                "%s: bad route count or capacity", who);
  VMAMD_REQUIRE(!expert_map || expert_map_len > 0, "%s: empty expert_map", who);
  VMAMD_REQUIRE(rows >= 0 && cols > 0 && cols % 128 == 0 && cols <= kRowThreads * 8 * kRowChunks,
                "%s: cols must be a multiple of 128 and at most %d", who, kRowThreads * 8 * kRowChunks);
  VMAMD_REQUIRE((topk_ids || numel == 0) && sorted && expert_ids && ntpp &&
                    ((x && xq && xs && xcorr) || rows == 0) &&
                    reinterpret_cast<uintptr_t>(x) % 16 == 0 && (reinterpret_cast<uintptr_t>(xq) & 7) == 0,
                "%s: null or misaligned pointer", who);
  int64_t chunk;
  int groups;
  align_grid(numel, chunk, groups);
  groups = std::max(groups, 1);
  // One row per wave for rows of up to 2048 columns; longer rows keep four
  // 256-thread rows per workgroup (at H = 4096, T = 4096 the wave form
  // measured 31.4 against 25.8 us: 16 rows per workgroup leave too few
  // workgroups in flight).
  const int cpl0 = static_cast<int>((cols + 511) / 512);
  const int cpl = cpl0 <= 4 ? cpl0 : 0;
  const int rows_per_block = cpl > 0 ? kAlignThreads / kWave : kAlignThreads / kRowThreads;
  const int64_t qblocks = (rows + rows_per_block - 1) / rows_per_block;
  W4ScalesT t{};
  int64_t trows = 0;
  if (sct) {
    t = *sct;
    for (int m = 0; m < 2; ++m) {
      VMAMD_REQUIRE(!t.in[m] || (t.out[m] && t.kp[m] > 0 && t.kp[m] % 2 == 0 &&
                                 reinterpret_cast<uintptr_t>(t.in[m]) % 8 == 0),
                    "%s: weight scales must be 8-byte aligned with an even count of word pairs per row", who);
      if (t.in[m]) trows += static_cast<int64_t>(t.E) * t.n[m];
    }
  }
  const int64_t tblocks = (trows + kAlignThreads - 1) / kAlignThreads;
  const dim3 grid(static_cast<unsigned>(groups + qblocks + tblocks));
#define VMAMD_ARQ(C)                                                                              \
  moe_align_rowquant_kernel<C><<<grid, kAlignThreads, 0, st>>>(                                   \
      topk_ids, numel, chunk, groups, num_experts, block_size, expert_map, expert_map_len, sorted, \
      capacity, expert_ids, ntpp, offsets, active, num_active, static_cast<const uint16_t*>(x),     \
      rows, static_cast<int>(cols), xq, xs, xcorr, static_cast<int>(qblocks), t)
  switch (cpl) {
    case 1: VMAMD_ARQ(1); break;
    case 2: VMAMD_ARQ(2); break;
    case 3: VMAMD_ARQ(3); break;
    case 4: VMAMD_ARQ(4); break;
    default: VMAMD_ARQ(0); break;
  }
#undef VMAMD_ARQ
  return check_launch(who);
}
}  // namespace vmamd

extern "C" int vmamd_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int num_experts,
                                          int block_size, const int32_t* expert_map,
                                          int64_t expert_map_len, int32_t* sorted_token_ids,
                                          int64_t capacity, int32_t* expert_ids,
                                          int32_t* num_tokens_post_pad, int32_t* expert_offsets,
                                          int32_t* scatter_idx, int32_t* active_experts,
                                          int32_t* num_active, vmamd_stream_t stream) {
  VMAMD_REQUIRE(num_experts > 0 && num_experts <= kMaxAlignExperts,
                "moe_align_block_size: num_experts must be in [1, %d] (got %d)", kMaxAlignExperts,
                num_experts);
  VMAMD_REQUIRE(block_size > 0, "moe_align_block_size: block_size must be positive");
  VMAMD_REQUIRE(numel >= 0 && numel < (1ll << 31) - 1, "moe_align_block_size: bad numel %lld",
                (long long)numel);
  VMAMD_REQUIRE(capacity >= numel + static_cast<int64_t>(num_experts) * (block_size - 1),
                "moe_align_block_size: capacity %lld < numel + num_experts * (block_size - 1) = %lld",
                (long long)capacity,
                (long long)(numel + static_cast<int64_t>(num_experts) * (block_size - 1)));
  VMAMD_REQUIRE(capacity < (1ll << 31), "moe_align_block_size: capacity too large");
  VMAMD_REQUIRE(!expert_map || expert_map_len > 0, "moe_align_block_size: empty expert_map");
  VMAMD_REQUIRE(!active_experts == !num_active,
                "moe_align_block_size: active_experts and num_active go together");
  VMAMD_REQUIRE((topk_ids || numel == 0) && sorted_token_ids && expert_ids && num_tokens_post_pad,
                "moe_align_block_size: null pointer");
  int64_t chunk;
  int groups;
  align_grid(numel, chunk, groups);
  moe_align_kernel<0><<<groups > 0 ? groups : 1, kAlignThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      topk_ids, numel, chunk, num_experts, block_size, expert_map, expert_map_len, sorted_token_ids,
      capacity, expert_ids, num_tokens_post_pad, expert_offsets, scatter_idx, active_experts,
      num_active, nullptr);
  return check_launch("moe_align_block_size");
}

extern "C" int vmamd_moe_align_block_size_quant_fp8(const int32_t* topk_ids, int64_t numel, int num_experts,
                                                    int block_size, const int32_t* expert_map,
                                                    int64_t expert_map_len, int32_t* sorted_token_ids,
                                                    int64_t capacity, int32_t* expert_ids,
                                                    int32_t* num_tokens_post_pad, int32_t* expert_offsets,
                                                    int32_t* active_experts, int32_t* num_active,
                                                    const void* x, int64_t rows, int64_t cols, void* xq,
                                                    float* xs, vmamd_stream_t stream) {
  VMAMD_REQUIRE(!active_experts == !num_active,
                "moe_align_block_size_quant_fp8: active_experts and num_active go together");
  return align_and_group_quant_fp8(topk_ids, numel, num_experts, block_size, expert_map, expert_map_len,
                                   sorted_token_ids, capacity, expert_ids, num_tokens_post_pad, expert_offsets,
                                   active_experts, num_active, x, rows, cols, static_cast<uint8_t*>(xq), xs,
                                   reinterpret_cast<hipStream_t>(stream));
}
