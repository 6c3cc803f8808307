// All-layer KV movement kernels: slot-to-slot move (tail-page copy-on-write),
// dense append (write_suffix_kv / set_kv_buffer) and page-table commit
// compaction (target_kv_commit).  Each is an HBM-bound copy of 16-byte
// vectors and one launch covers every layer.  Move and append: grid.y =
// layer * 2 + {K, V}, consecutive lanes move consecutive vectors of one token
// row.  Commit: one wave per (item, layer), its slots resolved once per wave
// through the page table.
#include "common.hpp"

namespace atlas {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

struct InlineItems {
  int64_t src[ATLAS_MAX_INLINE_ITEMS];
  int64_t dst[ATLAS_MAX_INLINE_ITEMS];
  int32_t req[ATLAS_MAX_INLINE_ITEMS];
};

// K[dst] <- K[src], V[dst] <- V[src] for every layer of the table.
__global__ __launch_bounds__(kThreads) void kv_move_kernel(LayerTable lt, SlotGeom g,
                                                           const int64_t* __restrict__ dst,
                                                           const int64_t* __restrict__ src,
                                                           int64_t n) {
  const int layer = blockIdx.y >> 1;
  char* base = const_cast<char*>((blockIdx.y & 1) ? lt.v[layer] : lt.k[layer]);
  const int64_t total = n * g.row_vecs;
  const int64_t first = int64_t(blockIdx.x) * kThreads * kUnroll + threadIdx.x;
  uint4 buf[kUnroll];
  int64_t dofs[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t idx = first + int64_t(u) * kThreads;
    dofs[u] = -1;
    if (idx < total) {
      int64_t item;
      int vec;
      split_row(idx, g, item, vec);
      const int64_t so = slot_offset(src[item], g) + vec_offset(vec, g);
      dofs[u] = slot_offset(dst[item], g) + vec_offset(vec, g);
      buf[u] = *reinterpret_cast<const uint4*>(base + so);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (dofs[u] >= 0) *reinterpret_cast<uint4*>(base + dofs[u]) = buf[u];
  }
}

// One wave per moved slot, for rows of CPR 1 KiB chunks (1 KiB and 2 KiB
// token rows).  The slot pair is wave-uniform and resolved to byte offsets
// once; the wave then copies the slot's K and V rows in every layer of the
// table, LB layers (2 * LB * CPR chunks per lane) in flight.  No branch splits
// a batch (a branch makes the compiler wait for every outstanding access,
// stores included, before each store): layers past the last one copy the last
// layer again, the same bytes to the same place.  dst and src slots are
// disjoint, so the copies of different waves never overlap.  The stores
// carry the non-temporal hint (the copies are not read again in this launch;
// 30.7 -> 24.1 us for a cold 94.6 MB copy-on-write); the loads do not, since
// a tail page's rows are the source of several copies and hit in L2.
template <int CPR, int LB>
__global__ __launch_bounds__(kThreads) void kv_move_rows_kernel(LayerTable lt, SlotGeom g, int num_layers,
                                                                const int64_t* __restrict__ dst,
                                                                const int64_t* __restrict__ src, int64_t n) {
  const int64_t item = int64_t(blockIdx.x) * (kThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (item >= n) return;
  const int lane = threadIdx.x & 63;
  const int64_t so = slot_offset(src[item], g) + int64_t(lane) * 16;
  const int64_t dof = slot_offset(dst[item], g) + int64_t(lane) * 16;
  for (int l0 = 0; l0 < num_layers; l0 += LB) {
    u32x4v buf[LB][2][CPR];
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int l = min(l0 + i, num_layers - 1);
      const char* kb = lt.k[l];
      const char* vb = lt.v[l];
#pragma unroll
      for (int c = 0; c < CPR; ++c) {
        buf[i][0][c] = *reinterpret_cast<const u32x4v*>(kb + so + c * 1024);
        buf[i][1][c] = *reinterpret_cast<const u32x4v*>(vb + so + c * 1024);
      }
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int l = min(l0 + i, num_layers - 1);
      char* kb = const_cast<char*>(lt.k[l]);
      char* vb = const_cast<char*>(lt.v[l]);
#pragma unroll
      for (int c = 0; c < CPR; ++c) {
        __builtin_nontemporal_store(buf[i][0][c], reinterpret_cast<u32x4v*>(kb + dof + c * 1024));
        __builtin_nontemporal_store(buf[i][1][c], reinterpret_cast<u32x4v*>(vb + dof + c * 1024));
      }
    }
  }
}

struct SrcTable {
  const char* k[ATLAS_MAX_LAYERS_PER_LAUNCH];
  const char* v[ATLAS_MAX_LAYERS_PER_LAUNCH];
};

// Dense rows -> slots, every layer.
__global__ __launch_bounds__(kThreads) void kv_append_kernel(LayerTable lt, SrcTable st, SlotGeom g,
                                                             int64_t src_token_stride,
                                                             const int64_t* __restrict__ dst,
                                                             int64_t dst_start, int64_t n) {
  const int layer = blockIdx.y >> 1;
  const bool is_v = blockIdx.y & 1;
  char* base = const_cast<char*>(is_v ? lt.v[layer] : lt.k[layer]);
  const char* sbase = is_v ? st.v[layer] : st.k[layer];
  const int64_t total = n * g.row_vecs;
  const int64_t first = int64_t(blockIdx.x) * kThreads * kUnroll + threadIdx.x;
  uint4 buf[kUnroll];
  int64_t dofs[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t idx = first + int64_t(u) * kThreads;
    dofs[u] = -1;
    if (idx < total) {
      int64_t item;
      int vec;
      split_row(idx, g, item, vec);
      const int64_t slot = dst ? dst[item] : dst_start + item;
      dofs[u] = slot_offset(slot, g) + vec_offset(vec, g);
      buf[u] = *reinterpret_cast<const uint4*>(sbase + item * src_token_stride + int64_t(vec) * 16);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (dofs[u] >= 0) *reinterpret_cast<uint4*>(base + dofs[u]) = buf[u];
  }
}

// Logical position of a request -> physical slot through its page table.
__device__ __forceinline__ int64_t position_slot(int64_t pos, int req, const int32_t* kv_indptr,
                                                 const int32_t* kv_indices, const SlotGeom& g) {
  if (kv_indices == nullptr) return pos;
  int64_t lp, off;
  if (g.page_shift >= 0) {
    lp = pos >> g.page_shift;
    off = pos & (g.page_size - 1);
  } else {
    lp = pos / g.page_size;
    off = pos - lp * g.page_size;
  }
  const int64_t base = kv_indptr ? kv_indptr[req] : 0;
  return int64_t(kv_indices[base + lp]) * g.page_size + off;
}

// Commit compaction modes.  kCopy: in place (no destination aliases another
// item's source).  kGather: rows -> workspace [layer][kv][item][row].
// kScatter: workspace -> destination rows.
enum CommitMode { kCopy = 0, kGather = 1, kScatter = 2 };

// Commit compaction, one wave per (item, layer): the item's positions, page
// table entries and slots are wave-uniform (scalar loads), and the wave moves
// the K row and the V row with every lane holding row_vecs/64 vectors of each
// in flight.  Block = 4 waves = 4 consecutive layers of one item.
constexpr int kRowWaves = 4;

// Loads and stores carry the non-temporal hint: each row is read once and
// written once (a cold 16 MiB commit of 32 requests: 10.1 -> 7.8 us).
// CPR: 1 KiB chunks per token row (1 or 2: every load of the row is issued
// before its stores, so a wave keeps its whole K and V rows in flight), or 0
// for other row sizes (a loop of 16-byte vectors).
template <int MODE, bool INLINE, int CPR>
__global__ __launch_bounds__(kThreads) void kv_commit_rows_kernel(
    LayerTable lt, SlotGeom g, int nl, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ kv_indices, const int32_t* __restrict__ item_req,
    const int64_t* __restrict__ src_pos, const int64_t* __restrict__ dst_pos, InlineItems items, int64_t n,
    char* __restrict__ ws, int layer0) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int layer = blockIdx.y * kRowWaves + wave;
  if (layer >= nl) return;
  const int lane = threadIdx.x & 63;
  const int64_t item = blockIdx.x;
  int req;
  int64_t sp, dp;
  if (INLINE) {
    req = items.req[item];
    sp = items.src[item];
    dp = items.dst[item];
  } else {
    req = item_req ? item_req[item] : 0;
    sp = src_pos[item];
    dp = dst_pos[item];
  }
  req = __builtin_amdgcn_readfirstlane(req);
  const int64_t row_bytes = int64_t(g.row_vecs) * 16;
  int64_t src_off = 0, dst_off = 0;
  if (MODE != kScatter) src_off = slot_offset(position_slot(sp, req, kv_indptr, kv_indices, g), g);
  if (MODE != kGather) dst_off = slot_offset(position_slot(dp, req, kv_indptr, kv_indices, g), g);
  const char* src_k;
  const char* src_v;
  char* dst_k;
  char* dst_v;
  {
    char* kb = const_cast<char*>(lt.k[layer]);
    char* vb = const_cast<char*>(lt.v[layer]);
    char* wk = ws ? ws + ((int64_t(layer0 + layer) * 2 + 0) * n + item) * row_bytes : nullptr;
    char* wv = ws ? ws + ((int64_t(layer0 + layer) * 2 + 1) * n + item) * row_bytes : nullptr;
    src_k = (MODE == kScatter) ? wk : kb + src_off;
    src_v = (MODE == kScatter) ? wv : vb + src_off;
    dst_k = (MODE == kGather) ? wk : kb + dst_off;
    dst_v = (MODE == kGather) ? wv : vb + dst_off;
  }
  // paged rows may be split by KV head; workspace rows are contiguous
  auto src_off_of = [&](int v) { return MODE == kScatter ? int64_t(v) * 16 : vec_offset(v, g); };
  auto dst_off_of = [&](int v) { return MODE == kGather ? int64_t(v) * 16 : vec_offset(v, g); };
  if constexpr (CPR > 0) {
    u32x4v a[CPR], b[CPR];
#pragma unroll
    for (int c = 0; c < CPR; ++c) {
      const int64_t so = src_off_of(c * 64 + lane);
      a[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(src_k + so));
      b[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(src_v + so));
    }
#pragma unroll
    for (int c = 0; c < CPR; ++c) {
      const int64_t d = dst_off_of(c * 64 + lane);
      __builtin_nontemporal_store(a[c], reinterpret_cast<u32x4v*>(dst_k + d));
      __builtin_nontemporal_store(b[c], reinterpret_cast<u32x4v*>(dst_v + d));
    }
  } else {
#pragma unroll 2
    for (int v = lane; v < g.row_vecs; v += 64) {
      const uint4 a = *reinterpret_cast<const uint4*>(src_k + src_off_of(v));
      const uint4 b = *reinterpret_cast<const uint4*>(src_v + src_off_of(v));
      *reinterpret_cast<uint4*>(dst_k + dst_off_of(v)) = a;
      *reinterpret_cast<uint4*>(dst_v + dst_off_of(v)) = b;
    }
  }
}

int make_geom(int64_t page_size, int64_t page_stride, int64_t token_stride, int64_t row_bytes,
              SlotGeom& g, int64_t head_bytes = 0, int64_t head_stride = 0) {
  ATLAS_REQUIRE(page_size > 0, "page_size must be positive");
  ATLAS_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0, "row_bytes must be a positive multiple of 16");
  ATLAS_REQUIRE(page_stride % 16 == 0 && token_stride % 16 == 0,
                "page and token strides must be multiples of 16 bytes");
  ATLAS_REQUIRE(row_bytes / 16 < (int64_t(1) << 30), "row_bytes too large");
  g.page_stride = page_stride;
  g.token_stride = token_stride;
  g.page_size = page_size;
  g.page_shift = ilog2_exact(page_size);
  g.row_vecs = static_cast<int32_t>(row_bytes / 16);
  g.row_shift = ilog2_exact(g.row_vecs);
  g.head_shift = -1;
  g.head_stride = 0;
  if (head_stride != 0 && head_stride != head_bytes) {
    // rows split by KV head: head_bytes contiguous per head, head_stride apart
    ATLAS_REQUIRE(head_bytes > 0 && head_bytes % 16 == 0 && row_bytes % head_bytes == 0,
                  "head_bytes must be a positive multiple of 16 dividing row_bytes");
    ATLAS_REQUIRE(ilog2_exact(head_bytes / 16) >= 0, "head_bytes / 16 must be a power of two");
    ATLAS_REQUIRE(head_stride % 16 == 0 && head_stride >= head_bytes,
                  "head_stride must be a multiple of 16 bytes covering a head's row");
    g.head_shift = ilog2_exact(head_bytes / 16);
    g.head_stride = head_stride;
  }
  return ATLAS_OK;
}

int check_layers(const void* const* k_layers, const void* const* v_layers, int num_layers) {
  ATLAS_REQUIRE(num_layers > 0, "num_layers must be positive");
  ATLAS_REQUIRE(k_layers != nullptr && v_layers != nullptr, "layer tables must not be NULL");
  for (int i = 0; i < num_layers; ++i) {
    ATLAS_REQUIRE(k_layers[i] != nullptr && v_layers[i] != nullptr, "layer %d base is NULL", i);
    ATLAS_REQUIRE((reinterpret_cast<uintptr_t>(k_layers[i]) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(v_layers[i]) & 15) == 0,
                  "layer %d base is not 16-byte aligned", i);
  }
  return ATLAS_OK;
}

void fill_table(LayerTable& lt, const void* const* k_layers, const void* const* v_layers, int l0,
                int nl) {
  for (int i = 0; i < ATLAS_MAX_LAYERS_PER_LAUNCH; ++i) {
    lt.k[i] = i < nl ? static_cast<const char*>(k_layers[l0 + i]) : nullptr;
    lt.v[i] = i < nl ? static_cast<const char*>(v_layers[l0 + i]) : nullptr;
  }
}

dim3 copy_grid(int64_t n, const SlotGeom& g, int nl) {
  const int64_t total = n * g.row_vecs;
  const int64_t per_block = int64_t(kThreads) * kUnroll;
  return dim3(static_cast<unsigned>((total + per_block - 1) / per_block), static_cast<unsigned>(2 * nl));
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" int atlas_kv_move_slots(const void* const* k_layers, const void* const* v_layers,
                                   int num_layers, int64_t page_size, int64_t page_stride,
                                   int64_t token_stride, int64_t row_bytes,
                                   const int64_t* dst_slots_dev, const int64_t* src_slots_dev,
                                   int64_t n, void* stream) {
  ATLAS_REQUIRE(n >= 0, "n must be non-negative");
  if (n == 0) return ATLAS_OK;
  ATLAS_REQUIRE(dst_slots_dev && src_slots_dev, "slot arrays must not be NULL");
  int rc = check_layers(k_layers, v_layers, num_layers);
  if (rc) return rc;
  SlotGeom g;
  if ((rc = make_geom(page_size, page_stride, token_stride, row_bytes, g))) return rc;
  for (int l0 = 0; l0 < num_layers; l0 += ATLAS_MAX_LAYERS_PER_LAUNCH) {
    const int nl = std::min(ATLAS_MAX_LAYERS_PER_LAUNCH, num_layers - l0);
    LayerTable lt;
    fill_table(lt, k_layers, v_layers, l0, nl);
    if (g.row_vecs == 64 || g.row_vecs == 128) {
      // 1 KiB or 2 KiB token rows: one wave per slot, all layers
      const dim3 grid(static_cast<unsigned>((n + kThreads / 64 - 1) / (kThreads / 64)));
      if (g.row_vecs == 64)
        hipLaunchKernelGGL((kv_move_rows_kernel<1, 8>), grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                           lt, g, nl, dst_slots_dev, src_slots_dev, n);
      else
        hipLaunchKernelGGL((kv_move_rows_kernel<2, 4>), grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                           lt, g, nl, dst_slots_dev, src_slots_dev, n);
      if ((rc = launch_status("kv_move_rows_kernel"))) return rc;
      continue;
    }
    hipLaunchKernelGGL(kv_move_kernel, copy_grid(n, g, nl), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), lt, g, dst_slots_dev, src_slots_dev, n);
    if ((rc = launch_status("kv_move_kernel"))) return rc;
  }
  return ATLAS_OK;
}

extern "C" int atlas_kv_append(const void* const* k_layers, const void* const* v_layers,
                               int num_layers, int64_t page_size, int64_t page_stride,
                               int64_t token_stride, int64_t row_bytes, int64_t head_bytes,
                               int64_t head_stride, const void* const* k_src,
                               const void* const* v_src, int64_t src_token_stride,
                               const int64_t* dst_slots_dev, int64_t dst_start, int64_t n,
                               void* stream) {
  ATLAS_REQUIRE(n >= 0, "n must be non-negative");
  if (n == 0) return ATLAS_OK;
  int rc = check_layers(k_layers, v_layers, num_layers);
  if (rc) return rc;
  if ((rc = check_layers(k_src, v_src, num_layers))) return rc;
  ATLAS_REQUIRE(src_token_stride % 16 == 0 && src_token_stride >= row_bytes,
                "source token stride must be a multiple of 16 bytes and cover a row");
  ATLAS_REQUIRE(dst_slots_dev != nullptr || dst_start >= 0, "dst_start must be non-negative");
  SlotGeom g;
  if ((rc = make_geom(page_size, page_stride, token_stride, row_bytes, g, head_bytes, head_stride))) return rc;
  for (int l0 = 0; l0 < num_layers; l0 += ATLAS_MAX_LAYERS_PER_LAUNCH) {
    const int nl = std::min(ATLAS_MAX_LAYERS_PER_LAUNCH, num_layers - l0);
    LayerTable lt;
    fill_table(lt, k_layers, v_layers, l0, nl);
    SrcTable st;
    for (int i = 0; i < ATLAS_MAX_LAYERS_PER_LAUNCH; ++i) {
      st.k[i] = i < nl ? static_cast<const char*>(k_src[l0 + i]) : nullptr;
      st.v[i] = i < nl ? static_cast<const char*>(v_src[l0 + i]) : nullptr;
    }
    hipLaunchKernelGGL(kv_append_kernel, copy_grid(n, g, nl), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), lt, st, g, src_token_stride, dst_slots_dev,
                       dst_start, n);
    if ((rc = launch_status("kv_append_kernel"))) return rc;
  }
  return ATLAS_OK;
}

namespace atlas {
namespace {

template <bool INLINE, int MODE>
void launch_commit_mode(int cpr, dim3 grid, hipStream_t stream, const LayerTable& lt, const SlotGeom& g, int nl,
                        const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* item_req,
                        const int64_t* src_pos, const int64_t* dst_pos, const InlineItems& items, int64_t n,
                        char* ws, int l0) {
  if (cpr == 1)
    hipLaunchKernelGGL((kv_commit_rows_kernel<MODE, INLINE, 1>), grid, dim3(kThreads), 0, stream, lt, g, nl,
                       kv_indptr, kv_indices, item_req, src_pos, dst_pos, items, n, ws, l0);
  else if (cpr == 2)
    hipLaunchKernelGGL((kv_commit_rows_kernel<MODE, INLINE, 2>), grid, dim3(kThreads), 0, stream, lt, g, nl,
                       kv_indptr, kv_indices, item_req, src_pos, dst_pos, items, n, ws, l0);
  else
    hipLaunchKernelGGL((kv_commit_rows_kernel<MODE, INLINE, 0>), grid, dim3(kThreads), 0, stream, lt, g, nl,
                       kv_indptr, kv_indices, item_req, src_pos, dst_pos, items, n, ws, l0);
}

template <bool INLINE>
void launch_commit_rows(int mode, int cpr, dim3 grid, hipStream_t stream, const LayerTable& lt, const SlotGeom& g,
                        int nl, const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* item_req,
                        const int64_t* src_pos, const int64_t* dst_pos, const InlineItems& items, int64_t n,
                        char* ws, int l0) {
  if (mode == kCopy)
    launch_commit_mode<INLINE, kCopy>(cpr, grid, stream, lt, g, nl, kv_indptr, kv_indices, item_req, src_pos,
                                      dst_pos, items, n, ws, l0);
  else if (mode == kGather)
    launch_commit_mode<INLINE, kGather>(cpr, grid, stream, lt, g, nl, kv_indptr, kv_indices, item_req, src_pos,
                                        dst_pos, items, n, ws, l0);
  else
    launch_commit_mode<INLINE, kScatter>(cpr, grid, stream, lt, g, nl, kv_indptr, kv_indices, item_req, src_pos,
                                         dst_pos, items, n, ws, l0);
}

template <bool INLINE>
int commit_impl(const void* const* k_layers, const void* const* v_layers, int num_layers,
                const SlotGeom& g, const int32_t* kv_indptr, const int32_t* kv_indices,
                const int32_t* item_req, const int64_t* src_pos, const int64_t* dst_pos,
                const InlineItems& items, int64_t n, bool staging, char* ws, hipStream_t stream) {
  int rc;
  // Staging gathers every layer before any scatter so no destination write can
  // precede a read of the same row.
  const int passes = staging ? 2 : 1;
  for (int pass = 0; pass < passes; ++pass) {
    for (int l0 = 0; l0 < num_layers; l0 += ATLAS_MAX_LAYERS_PER_LAUNCH) {
      const int nl = std::min(ATLAS_MAX_LAYERS_PER_LAUNCH, num_layers - l0);
      LayerTable lt;
      fill_table(lt, k_layers, v_layers, l0, nl);
      const dim3 grid(static_cast<unsigned>(n), static_cast<unsigned>((nl + kRowWaves - 1) / kRowWaves));
      const int mode = !staging ? kCopy : (pass == 0 ? kGather : kScatter);
      const int cpr = g.row_vecs == 64 ? 1 : (g.row_vecs == 128 ? 2 : 0);
      launch_commit_rows<INLINE>(mode, cpr, grid, stream, lt, g, nl, kv_indptr, kv_indices, item_req, src_pos,
                                 dst_pos, items, n, ws, l0);
      if ((rc = launch_status("kv_commit_kernel"))) return rc;
    }
  }
  return ATLAS_OK;
}

}  // namespace
}  // namespace atlas

extern "C" int atlas_kv_commit_paged(const void* const* k_layers, const void* const* v_layers,
                                     int num_layers, int64_t page_size, int64_t page_stride,
                                     int64_t token_stride, int64_t row_bytes, int64_t head_bytes,
                                     int64_t head_stride,
                                     const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev,
                                     const int32_t* item_req_dev, const int64_t* src_pos_dev,
                                     const int64_t* dst_pos_dev, int64_t n, int needs_staging,
                                     void* workspace_dev, size_t workspace_bytes, void* stream) {
  ATLAS_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "n must be in [0, 2^31)");
  if (n == 0) return ATLAS_OK;
  ATLAS_REQUIRE(src_pos_dev && dst_pos_dev, "position arrays must not be NULL");
  int rc = check_layers(k_layers, v_layers, num_layers);
  if (rc) return rc;
  SlotGeom g;
  if ((rc = make_geom(page_size, page_stride, token_stride, row_bytes, g, head_bytes, head_stride))) return rc;
  if (needs_staging) {
    const size_t need = size_t(n) * 2 * size_t(num_layers) * size_t(row_bytes);
    ATLAS_REQUIRE(workspace_dev != nullptr && workspace_bytes >= need,
                  "commit staging needs %zu workspace bytes, got %zu", need, workspace_bytes);
  }
  InlineItems unused{};
  return commit_impl<false>(k_layers, v_layers, num_layers, g, kv_indptr_dev, kv_indices_dev,
                            item_req_dev, src_pos_dev, dst_pos_dev, unused, n, needs_staging != 0,
                            static_cast<char*>(workspace_dev), static_cast<hipStream_t>(stream));
}

extern "C" int atlas_kv_commit_paged_host(const void* const* k_layers, const void* const* v_layers,
                                          int num_layers, int64_t page_size, int64_t page_stride,
                                          int64_t token_stride, int64_t row_bytes, int64_t head_bytes,
                                          int64_t head_stride,
                                          const int32_t* kv_indptr_dev,
                                          const int32_t* kv_indices_dev,
                                          const int32_t* item_req_host, const int64_t* src_pos_host,
                                          const int64_t* dst_pos_host, int64_t n, void* stream) {
  ATLAS_REQUIRE(n >= 0 && n <= ATLAS_MAX_INLINE_ITEMS, "inline commit takes 0..%d items, got %lld",
                ATLAS_MAX_INLINE_ITEMS, static_cast<long long>(n));
  if (n == 0) return ATLAS_OK;
  ATLAS_REQUIRE(src_pos_host && dst_pos_host, "position arrays must not be NULL");
  int rc = check_layers(k_layers, v_layers, num_layers);
  if (rc) return rc;
  SlotGeom g;
  if ((rc = make_geom(page_size, page_stride, token_stride, row_bytes, g, head_bytes, head_stride))) return rc;
  InlineItems items{};
  for (int64_t i = 0; i < n; ++i) {
    ATLAS_REQUIRE(src_pos_host[i] >= 0 && dst_pos_host[i] >= 0, "positions must be non-negative");
    items.src[i] = src_pos_host[i];
    items.dst[i] = dst_pos_host[i];
    items.req[i] = item_req_host ? item_req_host[i] : 0;
  }
  // A destination equal to another item's source (same request) would race in
  // one pass; the inline form has no staging buffer, so it rejects that case
  // and the caller uses atlas_kv_commit_paged with a workspace.
  for (int64_t i = 0; i < n; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      ATLAS_REQUIRE(i == j || items.req[i] != items.req[j] || items.dst[i] != items.src[j],
                    "commit destination %lld aliases the source of item %lld; use the staged form",
                    static_cast<long long>(i), static_cast<long long>(j));
    }
  }
  return commit_impl<true>(k_layers, v_layers, num_layers, g, kv_indptr_dev, kv_indices_dev, nullptr,
                           nullptr, nullptr, items, n, false, nullptr,
                           static_cast<hipStream_t>(stream));
}
