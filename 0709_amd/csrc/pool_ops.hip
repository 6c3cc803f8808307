// Page-pool bookkeeping kernels: reachability prune with an ascending
// free-list compaction, page ownership marking, paged-metadata compression of
// slot paths, and the decode / extend slot assignment of the paged allocator.
#include "common.hpp"

namespace atlas {
namespace {

constexpr int kSweepThreads = 1024;

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t value) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x)
    p[i] = value;
}

// Slot paths list the slots of a page consecutively, so only the first slot
// of each run of same-page slots sets the bit (one atomic per page run, not
// per slot).
__global__ void mark_pages_kernel(uint32_t* bitmap, int64_t num_pages, const int64_t* slots, int64_t n,
                                  int64_t page_size) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t s = slots[i];
    if (s < 0) continue;
    const int64_t page = s / page_size;
    if (page >= num_pages) continue;
    if (i > 0) {
      const int64_t prev = slots[i - 1];
      if (prev >= 0 && prev / page_size == page) continue;
    }
    atomicOr(&bitmap[page >> 5], 1u << (page & 31));
  }
}

// One workgroup: free = owned & ~live in ascending page order, owned &= live.
// Each thread owns a contiguous run of words; a block-wide exclusive scan of
// the per-thread counts gives every thread its output offset.
__global__ __launch_bounds__(kSweepThreads) void sweep_kernel(uint32_t* owned, const uint32_t* live,
                                                              int64_t num_words,
                                                              int64_t* free_pages,
                                                              int64_t* free_count) {
  __shared__ int64_t scan[kSweepThreads];
  const int tid = threadIdx.x;
  const int64_t per = (num_words + kSweepThreads - 1) / kSweepThreads;
  const int64_t w0 = min(num_words, int64_t(tid) * per);
  const int64_t w1 = min(num_words, w0 + per);
  int64_t cnt = 0;
  for (int64_t w = w0; w < w1; ++w) cnt += __popc(owned[w] & ~live[w]);
  scan[tid] = cnt;
  __syncthreads();
  for (int off = 1; off < kSweepThreads; off <<= 1) {
    const int64_t add = tid >= off ? scan[tid - off] : 0;
    __syncthreads();
    scan[tid] += add;
    __syncthreads();
  }
  int64_t pos = scan[tid] - cnt;
  for (int64_t w = w0; w < w1; ++w) {
    const uint32_t ow = owned[w];
    const uint32_t lv = live[w];
    uint32_t rel = ow & ~lv;
    while (rel) {
      const int b = __ffs(rel) - 1;
      free_pages[pos++] = w * 32 + b;
      rel &= rel - 1;
    }
    owned[w] = ow & lv;
  }
  if (tid == kSweepThreads - 1) *free_count = scan[tid];
}

// Mark and sweep in one workgroup for pools whose live bitmap fits in LDS
// (kFusedWords words): the live bits are set with LDS atomics (the marking
// rule of mark_pages_kernel), then the sweep of sweep_kernel reads them from
// LDS.  The live bitmap is also written out, as the three-launch path leaves
// it.  Each thread takes up to kFusedBatch slots, all loaded before the first
// atomic.  Larger slot lists go to the marking grid: one workgroup marking
// tens of thousands of slots measured slower than the three launches.
constexpr int64_t kFusedWords = 16384;
constexpr int kFusedBatch = 4;
constexpr int64_t kFusedMaxSlots = int64_t(kSweepThreads) * kFusedBatch;

// Sweep phase of the one-workgroup prunes: `live` (LDS) holds the marked
// pages; every owned page not live is released in ascending order (a scan of
// per-thread counts over contiguous word ranges gives each thread its output
// position), owned keeps owned & live, and the live bitmap is written out.
__device__ __forceinline__ void fused_sweep(uint32_t* owned, uint32_t* live_out, const uint32_t* live,
                                            int64_t num_words, int64_t* scan, int64_t* free_pages,
                                            int64_t* free_count) {
  const int tid = threadIdx.x;
  const int64_t per = (num_words + kSweepThreads - 1) / kSweepThreads;
  const int64_t w0 = min(num_words, int64_t(tid) * per);
  const int64_t w1 = min(num_words, w0 + per);
  int64_t cnt = 0;
  for (int64_t w = w0; w < w1; ++w) cnt += __popc(owned[w] & ~live[w]);
  scan[tid] = cnt;
  __syncthreads();
  for (int off = 1; off < kSweepThreads; off <<= 1) {
    const int64_t add = tid >= off ? scan[tid - off] : 0;
    __syncthreads();
    scan[tid] += add;
    __syncthreads();
  }
  int64_t pos = scan[tid] - cnt;
  for (int64_t w = w0; w < w1; ++w) {
    const uint32_t ow = owned[w];
    const uint32_t lv = live[w];
    uint32_t rel = ow & ~lv;
    while (rel) {
      const int b = __ffs(rel) - 1;
      free_pages[pos++] = w * 32 + b;
      rel &= rel - 1;
    }
    owned[w] = ow & lv;
    live_out[w] = lv;
  }
  if (tid == kSweepThreads - 1) *free_count = scan[tid];
}

__device__ __forceinline__ int64_t page_of(int64_t slot, int64_t page_size, int page_shift) {
  return page_shift >= 0 ? slot >> page_shift : slot / page_size;
}

__global__ __launch_bounds__(kSweepThreads) void prune_fused_kernel(uint32_t* owned, uint32_t* live_out,
                                                                    int64_t num_pages, int64_t num_words,
                                                                    const int64_t* slots, int64_t n,
                                                                    int64_t page_size, int page_shift,
                                                                    int64_t* free_pages, int64_t* free_count) {
  __shared__ uint32_t live[kFusedWords];
  __shared__ int64_t scan[kSweepThreads];
  const int tid = threadIdx.x;
  for (int64_t w = tid; w < num_words; w += kSweepThreads) live[w] = 0u;
  __syncthreads();
  {
    int64_t cur[kFusedBatch], prev[kFusedBatch];
#pragma unroll
    for (int k = 0; k < kFusedBatch; ++k) {
      const int64_t i = int64_t(k) * kSweepThreads + tid;
      cur[k] = i < n ? slots[i] : -1;
      prev[k] = (i > 0 && i < n) ? slots[i - 1] : -1;
    }
#pragma unroll
    for (int k = 0; k < kFusedBatch; ++k) {
      if (cur[k] < 0) continue;
      const int64_t page = page_of(cur[k], page_size, page_shift);
      if (page >= num_pages) continue;
      if (prev[k] >= 0 && page_of(prev[k], page_size, page_shift) == page) continue;
      atomicOr(&live[page >> 5], 1u << (page & 31));
    }
  }
  __syncthreads();
  fused_sweep(owned, live_out, live, num_words, scan, free_pages, free_count);
}

// The live paths of a prune by paths, by value in the kernel arguments.
struct PrunePaths {
  atlas_slot_path_t p[ATLAS_PRUNE_MAX_PATHS];
};

// Prune whose live slots are sampled from slot paths in the kernel: path p
// contributes slots[0], slots[ps], slots[2 ps], ... and, when bit p of
// last_mask is set, slots[len - 1] -- one slot of every page of a path laid
// out in whole pages.  Then the sweep of prune_fused_kernel.
// The int64 values of up to ATLAS_GATHER_MAX_SEGMENTS strided segments,
// concatenated into out (device memory or mapped host memory): one launch
// brings a pool's small results (released-page counts, page starts, check
// words) to the host together.
struct GatherSegments {
  atlas_i64_segment_t s[ATLAS_GATHER_MAX_SEGMENTS];
  int64_t start[ATLAS_GATHER_MAX_SEGMENTS + 1];
  int32_t n;
};

__device__ __forceinline__ void gather_values(const GatherSegments& g, int64_t* __restrict__ out, int64_t first,
                                              int64_t step) {
  const int64_t total = g.start[g.n];
  for (int64_t i = first; i < total; i += step) {
    int k = 0;
    while (i >= g.start[k + 1]) ++k;
    out[i] = g.s[k].src[(i - g.start[k]) * g.s[k].stride];
  }
}

__global__ __launch_bounds__(256) void gather_i64_kernel(const GatherSegments g, int64_t* __restrict__ out) {
  gather_values(g, out, int64_t(blockIdx.x) * blockDim.x + threadIdx.x, int64_t(gridDim.x) * blockDim.x);
}

__device__ __forceinline__ void prune_paths_body(uint32_t* owned, uint32_t* live_out,
                                                 int64_t num_pages, int64_t num_words, const PrunePaths& paths,
                                                 int num_paths, uint64_t last_mask, int64_t page_size,
                                                 int page_shift, int64_t* free_pages, int64_t* free_count) {
  __shared__ uint32_t live[kFusedWords];
  __shared__ int64_t scan[kSweepThreads];
  const int tid = threadIdx.x;
  for (int64_t w = tid; w < num_words; w += kSweepThreads) live[w] = 0u;
  __syncthreads();
  for (int p = 0; p < num_paths; ++p) {
    const int64_t* slots = paths.p[p].slots;
    const int64_t len = paths.p[p].len;
    if (len <= 0) continue;
    const int64_t starts = (len + page_size - 1) / page_size;
    const int64_t samples = starts + ((last_mask >> p) & 1ull);
    for (int64_t j = tid; j < samples; j += kSweepThreads) {
      const int64_t slot = slots[j < starts ? j * page_size : len - 1];
      if (slot < 0) continue;
      const int64_t page = page_of(slot, page_size, page_shift);
      if (page < num_pages) atomicOr(&live[page >> 5], 1u << (page & 31));
    }
  }
  __syncthreads();
  fused_sweep(owned, live_out, live, num_words, scan, free_pages, free_count);
}

__global__ __launch_bounds__(kSweepThreads) void prune_paths_kernel(uint32_t* owned, uint32_t* live_out,
                                                                    int64_t num_pages, int64_t num_words,
                                                                    PrunePaths paths, int num_paths,
                                                                    uint64_t last_mask, int64_t page_size,
                                                                    int page_shift, int64_t* free_pages,
                                                                    int64_t* free_count) {
  prune_paths_body(owned, live_out, num_pages, num_words, paths, num_paths, last_mask, page_size, page_shift,
                   free_pages, free_count);
}

// The same prune, then the workgroup copies the read-back segments to out:
// its own released-page count among them, read after the barrier that ends
// the sweep.
__global__ __launch_bounds__(kSweepThreads) void prune_paths_gather_kernel(
    uint32_t* owned, uint32_t* live_out, int64_t num_pages, int64_t num_words, PrunePaths paths, int num_paths,
    uint64_t last_mask, int64_t page_size, int page_shift, int64_t* free_pages, int64_t* free_count,
    const GatherSegments g, int64_t* __restrict__ out) {
  prune_paths_body(owned, live_out, num_pages, num_words, paths, num_paths, last_mask, page_size, page_shift,
                   free_pages, free_count);
  __syncthreads();
  gather_values(g, out, threadIdx.x, kSweepThreads);
}

// Page tables from concatenated slot paths.  Thread per page: the page id is
// the slot of the page's first token divided by page_size; the layout check
// requires that first slot to be page-aligned and every later slot of the page
// (within the path length) to follow it contiguously.
__global__ void paged_metadata_kernel(const int64_t* slots, const int64_t* path_offsets,
                                      const int64_t* page_offsets, int num_paths, int64_t total_pages,
                                      int64_t page_size, int validate, int32_t* page_indices,
                                      int32_t* layout_ok) {
  for (int64_t pg = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; pg < total_pages;
       pg += int64_t(gridDim.x) * blockDim.x) {
    // Binary search for the path owning this page.
    int lo = 0, hi = num_paths - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (page_offsets[mid] <= pg) lo = mid; else hi = mid - 1;
    }
    const int64_t local = pg - page_offsets[lo];
    const int64_t begin = path_offsets[lo] + local * page_size;
    const int64_t end = min(path_offsets[lo + 1], begin + page_size);
    const int64_t first = slots[begin];
    page_indices[pg] = static_cast<int32_t>(first >= 0 ? first / page_size : -((-first + page_size - 1) / page_size));
    if (validate) {
      bool ok = (((first % page_size) + page_size) % page_size) == 0;
      for (int64_t i = begin + 1; ok && i < end; ++i) ok = slots[i] == first + (i - begin);
      if (!ok) *layout_ok = 0;
    }
  }
}

// Decode slots: request i continues its tail page when (seq_len - 1) is not a
// page boundary, else takes the next page of the free list (in request order).
__global__ __launch_bounds__(1024) void alloc_decode_kernel(const int64_t* seq_lens, const int64_t* last_loc,
                                                            const int64_t* free_pages, int64_t page_size,
                                                            int bs, int64_t* out) {
  __shared__ int scan[1024];
  const int tid = threadIdx.x;
  int base = 0;
  for (int c0 = 0; c0 < bs; c0 += 1024) {
    const int i = c0 + tid;
    const int need = (i < bs && ((seq_lens[i] - 1) % page_size) == 0) ? 1 : 0;
    scan[tid] = need;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int add = tid >= off ? scan[tid - off] : 0;
      __syncthreads();
      scan[tid] += add;
      __syncthreads();
    }
    if (i < bs) out[i] = need ? free_pages[base + scan[tid] - 1] * page_size : last_loc[i] + 1;
    base += scan[1023];
    __syncthreads();
  }
}

// Extend slots: request i appends seq_lens[i] - prefix_lens[i] tokens; it first
// fills the free tail of its current page (continuing last_loc), then takes
// new pages from the free list in request order.  Output tokens are packed in
// request order.  Offsets come from block-wide scans of the per-request token
// and new-page counts, so the host uploads nothing.
__global__ __launch_bounds__(1024) void alloc_extend_kernel(const int64_t* prefix_lens, const int64_t* seq_lens,
                                                            const int64_t* last_loc, const int64_t* free_pages,
                                                            int64_t page_size, int bs, int64_t* out) {
  __shared__ int64_t scan_tok[1024];
  __shared__ int64_t scan_pg[1024];
  const int tid = threadIdx.x;
  int64_t tok_base = 0, pg_base = 0;
  for (int c0 = 0; c0 < bs; c0 += 1024) {
    const int i = c0 + tid;
    int64_t ntok = 0, npg = 0, pre = 0, seq = 0;
    if (i < bs) {
      pre = prefix_lens[i];
      seq = seq_lens[i];
      ntok = seq - pre;
      npg = (seq + page_size - 1) / page_size - (pre + page_size - 1) / page_size;
    }
    scan_tok[tid] = ntok;
    scan_pg[tid] = npg;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int64_t at = tid >= off ? scan_tok[tid - off] : 0;
      const int64_t ap = tid >= off ? scan_pg[tid - off] : 0;
      __syncthreads();
      scan_tok[tid] += at;
      scan_pg[tid] += ap;
      __syncthreads();
    }
    if (i < bs) {
      int64_t o = tok_base + scan_tok[tid] - ntok;
      int64_t pg = pg_base + scan_pg[tid] - npg;
      int64_t cur = last_loc[i];
      for (int64_t t = pre; t < seq; ++t) {
        const int64_t slot = (t % page_size == 0) ? free_pages[pg++] * page_size : cur + 1;
        out[o++] = slot;
        cur = slot;
      }
    }
    tok_base += scan_tok[1023];
    pg_base += scan_pg[1023];
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Frontier step of many requests: one workgroup per active route.
// ---------------------------------------------------------------------------
constexpr int kFrontierThreads = 256;

struct FrontierLimits {
  int64_t num_free;
  int64_t page_size;
  int64_t num_pages;
  int64_t req_rows;
  int64_t row_stride;
  int64_t flat_total;
  int64_t cow_total;
  int64_t page_total;
  int64_t num_routes;
};

__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

// Every index a descriptor carries stays inside the buffers the launch was
// given; a route that fails is skipped (and reported in its check word).
__device__ bool frontier_route_ok(const atlas_pool_frontier_route_t& d, const FrontierLimits& L) {
  const int64_t ps = L.page_size;
  if (d.prev_len < 0 || d.prev_len + 1 > L.row_stride) return false;
  if (d.prev_len > 0 && d.path == nullptr) return false;
  if (d.flat_offset < 0 || d.flat_offset + d.prev_len + 1 > L.flat_total) return false;
  const int64_t npages = (d.prev_len + ps) / ps;
  if (d.page_offset < 0 || d.page_offset + npages > L.page_total) return false;
  if (d.cow_tail != 0 && d.cow_tail != d.prev_len % ps) return false;
  if (d.cow_tail > 0 && (d.cow_free_index < 0 || d.cow_free_index >= L.num_free || d.cow_offset < 0 ||
                         d.cow_offset + d.cow_tail > L.cow_total))
    return false;
  if ((d.prev_len % ps == 0) != (d.new_free_index >= 0) || d.new_free_index >= L.num_free) return false;
  if (d.req_row < 0 || d.req_row >= L.req_rows || d.write_start < 0 || d.write_start > d.prev_len) return false;
  return d.group_first >= 0 && d.group_count >= 1 && d.group_first + d.group_count <= L.num_routes;
}

// Decode slot of a route (the allocator's decode rule applied to its new
// path) and the page its copy-on-write tail moves to (-1: none).
__device__ __forceinline__ int64_t frontier_decode_slot(const atlas_pool_frontier_route_t& d, const int64_t* free_pages,
                                                        int64_t ps, int64_t& cow_page) {
  cow_page = d.cow_tail > 0 ? free_pages[d.cow_free_index] : -1;
  if (d.new_free_index >= 0) return free_pages[d.new_free_index] * ps;
  const int64_t last = d.cow_tail > 0 ? cow_page * ps + (d.cow_tail - 1) : d.path[d.prev_len - 1];
  return last + 1;
}

// Slot p of the new path: the old path, its copied tail on the fresh page,
// then the decode slot.
__device__ __forceinline__ int64_t frontier_slot(const atlas_pool_frontier_route_t& d, int64_t p, int64_t cow_page,
                                                 int64_t out, int64_t ps) {
  if (p == d.prev_len) return out;
  const int64_t cut = d.prev_len - d.cow_tail;
  if (d.cow_tail > 0 && p >= cut) return cow_page * ps + (p - cut);
  return d.path[p];
}

// The route of this workgroup.  Writes its outputs and its check word
// (ATLAS_FRONTIER_* bits, 0 when every check passed), so nothing has to be
// cleared before the launch.  With batch != NULL it also writes the route's
// model inputs: token, sequence length, position, request row and route id,
// each a run of num_routes int64.
__device__ __forceinline__ void frontier_prepare_route(
    const atlas_pool_frontier_route_t* routes, const int64_t* tokens, const int64_t* route_ids,
    const FrontierLimits& L, const int64_t* __restrict__ free_pages, int64_t* __restrict__ req_to_token,
    int64_t* __restrict__ flat, int64_t* __restrict__ out_slots, int64_t* __restrict__ cow_dst,
    int64_t* __restrict__ cow_src, int32_t* __restrict__ kv_indptr, int32_t* __restrict__ kv_last,
    int32_t* __restrict__ seq_lens, int32_t* __restrict__ page_ids, int64_t* __restrict__ route_flags,
    int64_t* __restrict__ batch) {
  __shared__ int bits;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const atlas_pool_frontier_route_t d = routes[r];
  const int64_t ps = L.page_size;
  if (batch != nullptr && tid == 0) {
    const int64_t R = L.num_routes;
    batch[r] = tokens[r];
    batch[R + r] = d.prev_len + 1;
    batch[2 * R + r] = d.prev_len;
    batch[3 * R + r] = d.req_row;
    batch[4 * R + r] = route_ids[r];
  }
  if (!frontier_route_ok(d, L)) {
    if (tid == 0) route_flags[r] = ATLAS_FRONTIER_BAD_DESCRIPTOR;
    return;
  }
  if (tid == 0) bits = 0;
  int64_t cow_page;
  const int64_t out = frontier_decode_slot(d, free_pages, ps, cow_page);
  const int64_t n = d.prev_len + 1;
  const int64_t npages = (n + ps - 1) / ps;
  if (tid == 0) {
    out_slots[r] = out;
    seq_lens[r] = static_cast<int32_t>(n);
    kv_last[r] = static_cast<int32_t>(n - (npages - 1) * ps);
    kv_indptr[r + 1] = static_cast<int32_t>(d.page_offset + npages);
    if (r == 0) kv_indptr[0] = 0;
    if (d.owned_bitmap != nullptr) {
      const int64_t pg = floor_div(out, ps);
      if (pg >= 0 && pg < L.num_pages) atomicOr(&d.owned_bitmap[pg >> 5], 1u << (pg & 31));
      if (cow_page >= 0 && cow_page < L.num_pages) atomicOr(&d.owned_bitmap[cow_page >> 5], 1u << (cow_page & 31));
    }
  }
  int mine = 0;
  // New path, request-row slice, page table and layout check.
  for (int64_t p = tid; p < n; p += kFrontierThreads) {
    const int64_t v = frontier_slot(d, p, cow_page, out, ps);
    flat[d.flat_offset + p] = v;
    if (p >= d.write_start) req_to_token[d.req_row * L.row_stride + p] = v;
    const int64_t in_page = p % ps;
    if (in_page == 0) {
      page_ids[d.page_offset + p / ps] = static_cast<int32_t>(floor_div(v, ps));
      if (((v % ps) + ps) % ps != 0) mine |= ATLAS_FRONTIER_BAD_LAYOUT;
    } else if (v != frontier_slot(d, p - in_page, cow_page, out, ps) + in_page) {
      mine |= ATLAS_FRONTIER_BAD_LAYOUT;
    }
  }
  // Copy-on-write slot pairs; the fresh page must not be a copy source of
  // the same request.
  if (d.cow_tail > 0) {
    const int64_t cut = d.prev_len - d.cow_tail;
    for (int64_t t = tid; t < d.cow_tail; t += kFrontierThreads) {
      cow_dst[d.cow_offset + t] = cow_page * ps + t;
      cow_src[d.cow_offset + t] = d.path[cut + t];
    }
    // One thread per (route of the request, tail slot), so every descriptor
    // and tail load is in flight at once.
    const int64_t slots_per_route = ps;  // a tail holds fewer than page_size slots
    for (int64_t i = tid; i < d.group_count * slots_per_route; i += kFrontierThreads) {
      const int64_t s = d.group_first + i / slots_per_route;
      const int64_t t = i % slots_per_route;
      const atlas_pool_frontier_route_t e = routes[s];
      if (t >= e.cow_tail || !frontier_route_ok(e, L)) continue;
      if (floor_div(e.path[e.prev_len - e.cow_tail + t], ps) == cow_page) mine |= ATLAS_FRONTIER_COW_OVERLAP;
    }
  }
  // Distinct decode slots among the request's routes.
  for (int64_t s = d.group_first + tid; s < d.group_first + d.group_count; s += kFrontierThreads) {
    if (s == r) continue;
    const atlas_pool_frontier_route_t e = routes[s];
    if (!frontier_route_ok(e, L)) continue;
    int64_t ecow;
    if (frontier_decode_slot(e, free_pages, ps, ecow) == out) mine |= ATLAS_FRONTIER_DUPLICATE_SLOT;
  }
  __syncthreads();  // bits is cleared
  if (mine) atomicOr(&bits, mine);
  __syncthreads();
  if (tid == 0) route_flags[r] = bits;
}

__global__ __launch_bounds__(kFrontierThreads) void frontier_prepare_kernel(
    const atlas_pool_frontier_route_t* __restrict__ routes, FrontierLimits L, const int64_t* __restrict__ free_pages,
    int64_t* __restrict__ req_to_token, int64_t* __restrict__ flat, int64_t* __restrict__ out_slots,
    int64_t* __restrict__ cow_dst, int64_t* __restrict__ cow_src, int32_t* __restrict__ kv_indptr,
    int32_t* __restrict__ kv_last, int32_t* __restrict__ seq_lens, int32_t* __restrict__ page_ids,
    int64_t* __restrict__ route_flags) {
  frontier_prepare_route(routes, nullptr, nullptr, L, free_pages, req_to_token, flat, out_slots, cow_dst, cow_src,
                         kv_indptr, kv_last, seq_lens, page_ids, route_flags, nullptr);
}

// The descriptors, tokens and route ids of up to ATLAS_FRONTIER_MAX_HOST_ROUTES
// routes, passed by value in the launch's argument block.
struct FrontierHostRoutes {
  atlas_pool_frontier_route_t d[ATLAS_FRONTIER_MAX_HOST_ROUTES];
  int64_t token[ATLAS_FRONTIER_MAX_HOST_ROUTES];
  int64_t route_id[ATLAS_FRONTIER_MAX_HOST_ROUTES];
};

__global__ __launch_bounds__(kFrontierThreads) void frontier_prepare_host_kernel(
    const FrontierHostRoutes a, FrontierLimits L, const int64_t* __restrict__ free_pages,
    int64_t* __restrict__ req_to_token, int64_t* __restrict__ flat, int64_t* __restrict__ out_slots,
    int64_t* __restrict__ cow_dst, int64_t* __restrict__ cow_src, int32_t* __restrict__ kv_indptr,
    int32_t* __restrict__ kv_last, int32_t* __restrict__ seq_lens, int32_t* __restrict__ page_ids,
    int64_t* __restrict__ route_flags, int64_t* __restrict__ batch) {
  frontier_prepare_route(a.d, a.token, a.route_id, L, free_pages, req_to_token, flat, out_slots, cow_dst, cow_src,
                         kv_indptr, kv_last, seq_lens, page_ids, route_flags, batch);
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" int atlas_mark_pages(uint32_t* bitmap_dev, int64_t num_pages, const int64_t* slots_dev,
                                int64_t n, int64_t page_size, void* stream) {
  ATLAS_REQUIRE(bitmap_dev && num_pages > 0 && page_size > 0, "bad bitmap / page arguments");
  if (n <= 0) return ATLAS_OK;
  ATLAS_REQUIRE(slots_dev, "slots must not be NULL");
  const int blocks = static_cast<int>(std::min<int64_t>((n + 255) / 256, 1024));
  hipLaunchKernelGGL(mark_pages_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     bitmap_dev, num_pages, slots_dev, n, page_size);
  return launch_status("mark_pages_kernel");
}

extern "C" int atlas_prune_pages(uint32_t* owned_bitmap_dev, uint32_t* live_bitmap_dev, int64_t num_pages,
                                 const int64_t* live_slots_dev, int64_t n_live_slots, int64_t page_size,
                                 int64_t* free_pages_dev, int64_t* free_count_dev, void* stream) {
  ATLAS_REQUIRE(owned_bitmap_dev && live_bitmap_dev && free_pages_dev && free_count_dev,
                "prune buffers must not be NULL");
  ATLAS_REQUIRE(num_pages > 0 && page_size > 0, "num_pages and page_size must be positive");
  ATLAS_REQUIRE(n_live_slots == 0 || live_slots_dev, "live slots must not be NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t words = (num_pages + 31) / 32;
  if (words <= kFusedWords && n_live_slots <= kFusedMaxSlots) {
    hipLaunchKernelGGL(prune_fused_kernel, dim3(1), dim3(kSweepThreads), 0, s, owned_bitmap_dev,
                       live_bitmap_dev, num_pages, words, live_slots_dev, n_live_slots, page_size,
                       ilog2_exact(page_size), free_pages_dev,
                       free_count_dev);
    return launch_status("prune_fused_kernel");
  }
  const int fill_blocks = static_cast<int>(std::min<int64_t>((words + 255) / 256, 1024));
  hipLaunchKernelGGL(fill_u32_kernel, dim3(fill_blocks), dim3(256), 0, s, live_bitmap_dev, words, 0u);
  int rc = launch_status("fill_u32_kernel");
  if (rc) return rc;
  if (n_live_slots > 0) {
    const int blocks = static_cast<int>(std::min<int64_t>((n_live_slots + 255) / 256, 1024));
    hipLaunchKernelGGL(mark_pages_kernel, dim3(blocks), dim3(256), 0, s, live_bitmap_dev, num_pages,
                       live_slots_dev, n_live_slots, page_size);
    if ((rc = launch_status("mark_pages_kernel"))) return rc;
  }
  hipLaunchKernelGGL(sweep_kernel, dim3(1), dim3(kSweepThreads), 0, s, owned_bitmap_dev, live_bitmap_dev,
                     words, free_pages_dev, free_count_dev);
  return launch_status("sweep_kernel");
}

namespace {

// Arguments of the prune by paths, checked: ATLAS_OK, or the refusal.
int prune_paths_args(uint32_t* owned_bitmap_dev, uint32_t* live_bitmap_dev, int64_t num_pages,
                     const atlas_slot_path_t* paths, int num_paths, int64_t page_size, int64_t* free_pages_dev,
                     int64_t* free_count_dev, PrunePaths* pp) {
  ATLAS_REQUIRE(owned_bitmap_dev && live_bitmap_dev && free_pages_dev && free_count_dev,
                "prune buffers must not be NULL");
  ATLAS_REQUIRE(num_pages > 0 && page_size > 0, "num_pages and page_size must be positive");
  ATLAS_REQUIRE(num_paths >= 0 && (num_paths == 0 || paths), "paths must not be NULL");
  if (num_paths > ATLAS_PRUNE_MAX_PATHS || (num_pages + 31) / 32 > kFusedWords) {
    set_error("prune by paths takes at most %d paths and %lld pages (got %d, %lld)", ATLAS_PRUNE_MAX_PATHS,
              static_cast<long long>(kFusedWords * 32), num_paths, static_cast<long long>(num_pages));
    return ATLAS_EUNSUPPORTED;
  }
  for (int p = 0; p < num_paths; ++p) {
    ATLAS_REQUIRE(paths[p].len >= 0 && (paths[p].len == 0 || paths[p].slots), "path %d: bad slots or length", p);
    pp->p[p] = paths[p];
  }
  return ATLAS_OK;
}

// The read-back segments, checked, into the launch's argument block.
int gather_args(const atlas_i64_segment_t* segments_host, int num_segments, GatherSegments* g) {
  ATLAS_REQUIRE(num_segments >= 0 && num_segments <= ATLAS_GATHER_MAX_SEGMENTS, "num_segments must be in [0, %d]",
                ATLAS_GATHER_MAX_SEGMENTS);
  ATLAS_REQUIRE(num_segments == 0 || segments_host, "segments must not be NULL");
  g->n = num_segments;
  g->start[0] = 0;
  for (int k = 0; k < num_segments; ++k) {
    const atlas_i64_segment_t& sk = segments_host[k];
    ATLAS_REQUIRE(sk.count >= 0 && (sk.count == 0 || sk.src), "segment %d: bad source or count", k);
    g->s[k] = sk;
    g->start[k + 1] = g->start[k] + sk.count;
  }
  ATLAS_REQUIRE(g->start[num_segments] < (int64_t(1) << 31), "too many values");
  return ATLAS_OK;
}

}  // namespace

extern "C" int atlas_prune_pages_paths(uint32_t* owned_bitmap_dev, uint32_t* live_bitmap_dev, int64_t num_pages,
                                       const atlas_slot_path_t* paths, int num_paths, uint64_t last_slot_mask,
                                       int64_t page_size, int64_t* free_pages_dev, int64_t* free_count_dev,
                                       void* stream) {
  PrunePaths pp{};
  if (int rc = prune_paths_args(owned_bitmap_dev, live_bitmap_dev, num_pages, paths, num_paths, page_size,
                                free_pages_dev, free_count_dev, &pp))
    return rc;
  const int64_t words = (num_pages + 31) / 32;
  hipLaunchKernelGGL(prune_paths_kernel, dim3(1), dim3(kSweepThreads), 0, static_cast<hipStream_t>(stream),
                     owned_bitmap_dev, live_bitmap_dev, num_pages, words, pp, num_paths, last_slot_mask, page_size,
                     ilog2_exact(page_size), free_pages_dev, free_count_dev);
  return launch_status("prune_paths_kernel");
}

extern "C" int atlas_prune_pages_paths_gather(uint32_t* owned_bitmap_dev, uint32_t* live_bitmap_dev,
                                              int64_t num_pages, const atlas_slot_path_t* paths, int num_paths,
                                              uint64_t last_slot_mask, int64_t page_size, int64_t* free_pages_dev,
                                              int64_t* free_count_dev, const atlas_i64_segment_t* segments_host,
                                              int num_segments, int64_t* out, void* stream) {
  PrunePaths pp{};
  if (int rc = prune_paths_args(owned_bitmap_dev, live_bitmap_dev, num_pages, paths, num_paths, page_size,
                                free_pages_dev, free_count_dev, &pp))
    return rc;
  GatherSegments g{};
  if (int rc = gather_args(segments_host, num_segments, &g)) return rc;
  ATLAS_REQUIRE(g.start[num_segments] == 0 || out, "out must not be NULL");
  const int64_t words = (num_pages + 31) / 32;
  hipLaunchKernelGGL(prune_paths_gather_kernel, dim3(1), dim3(kSweepThreads), 0, static_cast<hipStream_t>(stream),
                     owned_bitmap_dev, live_bitmap_dev, num_pages, words, pp, num_paths, last_slot_mask, page_size,
                     ilog2_exact(page_size), free_pages_dev, free_count_dev, g, out);
  return launch_status("prune_paths_gather_kernel");
}

extern "C" int atlas_gather_i64(const atlas_i64_segment_t* segments_host, int num_segments, int64_t* out,
                                void* stream) {
  GatherSegments g{};
  if (int rc = gather_args(segments_host, num_segments, &g)) return rc;
  const int64_t total = g.start[num_segments];
  if (total == 0) return ATLAS_OK;
  ATLAS_REQUIRE(out, "out must not be NULL");
  const int blocks = static_cast<int>(std::min<int64_t>((total + 255) / 256, 64));
  hipLaunchKernelGGL(gather_i64_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), g, out);
  return launch_status("gather_i64_kernel");
}

extern "C" int atlas_paged_metadata(const int64_t* slots_dev, const int64_t* path_offsets_dev,
                                    const int64_t* page_offsets_dev, int num_paths, int64_t total_pages,
                                    int64_t page_size, int validate, int32_t* kv_page_indices_dev,
                                    int32_t* layout_ok_dev, void* stream) {
  ATLAS_REQUIRE(num_paths > 0 && page_size > 0, "num_paths and page_size must be positive");
  ATLAS_REQUIRE(slots_dev && path_offsets_dev && page_offsets_dev && kv_page_indices_dev,
                "metadata buffers must not be NULL");
  ATLAS_REQUIRE(!validate || layout_ok_dev, "validation needs a layout flag");
  if (total_pages <= 0) return ATLAS_OK;
  const int blocks = static_cast<int>(std::min<int64_t>((total_pages + 255) / 256, 2048));
  hipLaunchKernelGGL(paged_metadata_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     slots_dev, path_offsets_dev, page_offsets_dev, num_paths, total_pages, page_size,
                     validate, kv_page_indices_dev, layout_ok_dev);
  return launch_status("paged_metadata_kernel");
}

extern "C" int atlas_alloc_decode_slots(const int64_t* seq_lens_dev, const int64_t* last_loc_dev,
                                        const int64_t* free_pages_dev, int64_t page_size, int bs,
                                        int64_t* out_dev, void* stream) {
  ATLAS_REQUIRE(bs >= 0 && page_size > 0, "bad batch / page size");
  if (bs == 0) return ATLAS_OK;
  ATLAS_REQUIRE(seq_lens_dev && last_loc_dev && free_pages_dev && out_dev, "NULL buffer");
  hipLaunchKernelGGL(alloc_decode_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), seq_lens_dev,
                     last_loc_dev, free_pages_dev, page_size, bs, out_dev);
  return launch_status("alloc_decode_kernel");
}

extern "C" int atlas_alloc_extend_slots(const int64_t* prefix_lens_dev, const int64_t* seq_lens_dev,
                                        const int64_t* last_loc_dev, const int64_t* free_pages_dev,
                                        int64_t page_size, int bs, int64_t* out_dev, void* stream) {
  ATLAS_REQUIRE(bs >= 0 && page_size > 0, "bad batch / page size");
  if (bs == 0) return ATLAS_OK;
  ATLAS_REQUIRE(prefix_lens_dev && seq_lens_dev && last_loc_dev && free_pages_dev && out_dev, "NULL buffer");
  hipLaunchKernelGGL(alloc_extend_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                     prefix_lens_dev, seq_lens_dev, last_loc_dev, free_pages_dev, page_size, bs, out_dev);
  return launch_status("alloc_extend_kernel");
}

namespace {

int frontier_limits(int num_routes, const int64_t* free_pages_dev, int64_t num_free, int64_t page_size,
                    int64_t num_pages, int64_t* req_to_token_dev, int64_t req_rows, int64_t req_row_stride,
                    int64_t* flat_dev, int64_t flat_total, int64_t* out_slots_dev, int64_t* cow_dst_dev,
                    int64_t* cow_src_dev, int64_t cow_total, int32_t* kv_indptr_dev, int32_t* kv_last_page_len_dev,
                    int32_t* seq_lens_dev, int32_t* kv_page_indices_dev, int64_t page_total,
                    int64_t* route_flags_dev, FrontierLimits* L) {
  ATLAS_REQUIRE(req_to_token_dev && flat_dev && out_slots_dev && kv_indptr_dev && kv_last_page_len_dev &&
                    seq_lens_dev && kv_page_indices_dev && route_flags_dev,
                "frontier buffers must not be NULL");
  ATLAS_REQUIRE(num_free >= 0 && (num_free == 0 || free_pages_dev), "free list must not be NULL");
  ATLAS_REQUIRE(cow_total >= 0 && (cow_total == 0 || (cow_dst_dev && cow_src_dev)), "copy-on-write lists missing");
  ATLAS_REQUIRE(req_rows > 0 && req_row_stride > 0, "request-row pool must not be empty");
  ATLAS_REQUIRE(flat_total >= num_routes && page_total >= num_routes, "output sizes too small for %d routes",
                num_routes);
  *L = FrontierLimits{num_free, page_size, num_pages, req_rows, req_row_stride, flat_total, cow_total, page_total,
                      num_routes};
  return ATLAS_OK;
}

}  // namespace

extern "C" int atlas_pool_prepare_frontier(const atlas_pool_frontier_route_t* routes_dev, int num_routes,
                                      const int64_t* free_pages_dev, int64_t num_free, int64_t page_size,
                                      int64_t num_pages, int64_t* req_to_token_dev, int64_t req_rows,
                                      int64_t req_row_stride, int64_t* flat_dev, int64_t flat_total,
                                      int64_t* out_slots_dev, int64_t* cow_dst_dev, int64_t* cow_src_dev,
                                      int64_t cow_total, int32_t* kv_indptr_dev, int32_t* kv_last_page_len_dev,
                                      int32_t* seq_lens_dev, int32_t* kv_page_indices_dev, int64_t page_total,
                                      int64_t* route_flags_dev, void* stream) {
  ATLAS_REQUIRE(num_routes >= 0 && page_size > 0 && num_pages > 0, "bad route count / page arguments");
  if (num_routes == 0) return ATLAS_OK;
  ATLAS_REQUIRE(routes_dev, "frontier buffers must not be NULL");
  FrontierLimits L;
  if (int rc = frontier_limits(num_routes, free_pages_dev, num_free, page_size, num_pages, req_to_token_dev, req_rows,
                               req_row_stride, flat_dev, flat_total, out_slots_dev, cow_dst_dev, cow_src_dev,
                               cow_total, kv_indptr_dev, kv_last_page_len_dev, seq_lens_dev, kv_page_indices_dev,
                               page_total, route_flags_dev, &L))
    return rc;
  hipLaunchKernelGGL(frontier_prepare_kernel, dim3(num_routes), dim3(kFrontierThreads), 0,
                     static_cast<hipStream_t>(stream), routes_dev, L, free_pages_dev, req_to_token_dev, flat_dev,
                     out_slots_dev, cow_dst_dev, cow_src_dev, kv_indptr_dev, kv_last_page_len_dev, seq_lens_dev,
                     kv_page_indices_dev, route_flags_dev);
  return launch_status("frontier_prepare_kernel");
}

extern "C" int atlas_pool_prepare_frontier_host(
    const atlas_pool_frontier_route_t* routes_host, const int64_t* tokens_host, const int64_t* route_ids_host,
    int num_routes, const int64_t* free_pages_dev, int64_t num_free, int64_t page_size, int64_t num_pages,
    int64_t* req_to_token_dev, int64_t req_rows, int64_t req_row_stride, int64_t* flat_dev, int64_t flat_total,
    int64_t* out_slots_dev, int64_t* cow_dst_dev, int64_t* cow_src_dev, int64_t cow_total, int32_t* kv_indptr_dev,
    int32_t* kv_last_page_len_dev, int32_t* seq_lens_dev, int32_t* kv_page_indices_dev, int64_t page_total,
    int64_t* route_flags_dev, int64_t* batch_dev, void* stream) {
  ATLAS_REQUIRE(num_routes >= 0 && page_size > 0 && num_pages > 0, "bad route count / page arguments");
  if (num_routes == 0) return ATLAS_OK;
  if (num_routes > ATLAS_FRONTIER_MAX_HOST_ROUTES) {
    set_error("a frontier step with descriptors from host memory takes at most %d routes (got %d)",
              ATLAS_FRONTIER_MAX_HOST_ROUTES, num_routes);
    return ATLAS_EUNSUPPORTED;
  }
  ATLAS_REQUIRE(routes_host && tokens_host && route_ids_host && batch_dev, "frontier buffers must not be NULL");
  FrontierLimits L;
  if (int rc = frontier_limits(num_routes, free_pages_dev, num_free, page_size, num_pages, req_to_token_dev, req_rows,
                               req_row_stride, flat_dev, flat_total, out_slots_dev, cow_dst_dev, cow_src_dev,
                               cow_total, kv_indptr_dev, kv_last_page_len_dev, seq_lens_dev, kv_page_indices_dev,
                               page_total, route_flags_dev, &L))
    return rc;
  FrontierHostRoutes a{};
  std::memcpy(a.d, routes_host, sizeof(atlas_pool_frontier_route_t) * num_routes);
  std::memcpy(a.token, tokens_host, sizeof(int64_t) * num_routes);
  std::memcpy(a.route_id, route_ids_host, sizeof(int64_t) * num_routes);
  hipLaunchKernelGGL(frontier_prepare_host_kernel, dim3(num_routes), dim3(kFrontierThreads), 0,
                     static_cast<hipStream_t>(stream), a, L, free_pages_dev, req_to_token_dev, flat_dev,
                     out_slots_dev, cow_dst_dev, cow_src_dev, kv_indptr_dev, kv_last_page_len_dev, seq_lens_dev,
                     kv_page_indices_dev, route_flags_dev, batch_dev);
  return launch_status("frontier_prepare_host_kernel");
}
