// Host-side tree specification of a verify step: the route trie, every node's
// ancestor set and the packed buffer the step uploads in one copy (token ids,
// depths, mask words, indptrs, page table, the tree block of the dense mask).
// Pure host code: no device call.
//
// Follows flashinfer_full_verify.py:541-567 (one node per path position),
// 570-616 (the deduplicated trie: a node per unique token prefix, numbered
// route by route, depth by depth) and 655-739 (kv_len, pages, last page length,
// the identity page table and the ancestor mask of the spec).

#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace atlas {
namespace {

constexpr int64_t kMaxNodes = int64_t(1) << 20;

struct SpecSizes {
  int64_t nodes_max;
  int64_t words;     // int64 mask words in the buffer (all nodes)
  int64_t tiles;     // words per node when tile words are stored, else 0
  int64_t i32_count; // even
  int64_t bytes;
};

int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Sizes of the buffer for `nodes` nodes.
SpecSizes spec_sizes(int64_t nodes, int64_t prefix_len, int64_t page_size) {
  SpecSizes s{};
  s.nodes_max = nodes;
  const int64_t kv_len = prefix_len + nodes;
  const int64_t pages = ceil_div64(kv_len, page_size);
  if (nodes <= 64) {
    s.words = nodes;
  } else if (nodes <= ATLAS_TREE_TILE_MAX_NODES) {
    s.tiles = (kv_len - 1) / 64 - prefix_len / 64 + 1;
    s.words = nodes * s.tiles;
  }
  s.i32_count = 5 + pages + (1 + pages) % 2;
  s.bytes = 16 * nodes + 8 * s.words + 4 * s.i32_count + nodes * nodes;
  return s;
}

// Open-addressing map (parent node, token) -> node for the deduplicated trie.
struct ChildMap {
  std::vector<int64_t> token;
  std::vector<int32_t> parent;
  std::vector<int32_t> node;  // -1: empty
  uint64_t mask = 0;

  void reset(int64_t nodes) {
    uint64_t cap = 16;
    while (cap < uint64_t(2 * nodes)) cap <<= 1;
    if (node.size() < cap) {
      token.resize(cap);
      parent.resize(cap);
      node.resize(cap);
    }
    mask = cap - 1;
    std::fill(node.begin(), node.begin() + cap, -1);
  }

  // The node of (par, tok), inserting `fresh` when absent.
  int32_t find_or_insert(int32_t par, int64_t tok, int32_t fresh, bool& inserted) {
    uint64_t h = (uint64_t(tok) * 0x9E3779B97F4A7C15ull) ^ (uint64_t(uint32_t(par + 1)) * 0xC2B2AE3D27D4EB4Full);
    h ^= h >> 29;
    for (uint64_t i = h & mask;; i = (i + 1) & mask) {
      if (node[i] < 0) {
        token[i] = tok;
        parent[i] = par;
        node[i] = fresh;
        inserted = true;
        return fresh;
      }
      if (token[i] == tok && parent[i] == par) {
        inserted = false;
        return node[i];
      }
    }
  }
};

struct Scratch {
  ChildMap children;
  std::vector<int64_t> tok, dep;
  std::vector<uint64_t> anc;  // nodes x ancestor words
};

thread_local Scratch t_scratch;

}  // namespace
}  // namespace atlas

using atlas::SpecSizes;

extern "C" int64_t atlas_tree_spec_bytes(int32_t num_paths, int32_t depth, int64_t prefix_len, int32_t page_size) {
  if (num_paths <= 0 || depth <= 0 || prefix_len < 0 || page_size <= 0) return -1;
  const int64_t nodes = int64_t(num_paths) * depth;
  if (nodes > atlas::kMaxNodes) return -1;
  // The size grows with the node count within each mask-word regime (up to
  // 64 nodes, up to ATLAS_TREE_TILE_MAX_NODES, beyond), so the larger of the
  // undeduplicated count and the largest count with tile words bounds it.
  const int64_t tiled = std::min<int64_t>(nodes, ATLAS_TREE_TILE_MAX_NODES);
  return std::max(atlas::spec_sizes(nodes, prefix_len, page_size).bytes,
                  atlas::spec_sizes(tiled, prefix_len, page_size).bytes);
}

extern "C" int atlas_tree_spec_build(const int64_t* paths_host, int32_t num_paths, int32_t depth, int32_t dedup,
                                     int64_t prefix_len, int32_t page_size, uint8_t* out_host, int64_t out_bytes,
                                     int32_t* parents_host, int32_t* route_nodes_host, int64_t* info_host) {
  ATLAS_REQUIRE(num_paths > 0, "paths must not be empty");
  ATLAS_REQUIRE(depth > 0, "paths must contain at least one token");
  ATLAS_REQUIRE(prefix_len >= 0 && page_size > 0, "prefix_len must be >= 0 and page_size positive");
  ATLAS_REQUIRE(int64_t(num_paths) * depth <= atlas::kMaxNodes, "at most %lld tree nodes",
                static_cast<long long>(atlas::kMaxNodes));
  ATLAS_REQUIRE((prefix_len + int64_t(num_paths) * depth) / page_size < INT32_MAX, "too many pages");
  ATLAS_REQUIRE(paths_host && out_host && parents_host && info_host && (route_nodes_host || !dedup),
                "paths, out, parents, route_nodes and info must not be NULL");
  atlas::Scratch& sc = atlas::t_scratch;
  const int64_t n_max = int64_t(num_paths) * depth;
  if (int64_t(sc.tok.size()) < n_max) {
    sc.tok.resize(n_max);
    sc.dep.resize(n_max);
  }
  // 1. nodes in creation order; a node's parent always precedes it
  int32_t n = 0;
  if (dedup) sc.children.reset(n_max);
  for (int32_t p = 0; p < num_paths; ++p) {
    int32_t par = -1;
    for (int32_t d = 0; d < depth; ++d) {
      const int64_t tok = paths_host[int64_t(p) * depth + d];
      int32_t node = n;
      bool fresh = true;
      if (dedup) node = sc.children.find_or_insert(par, tok, n, fresh);
      if (fresh) {
        sc.tok[n] = tok;
        sc.dep[n] = d;
        parents_host[n] = par;
        ++n;
      }
      if (route_nodes_host) route_nodes_host[int64_t(p) * depth + d] = node;
      par = node;
    }
  }
  const SpecSizes sz = atlas::spec_sizes(n, prefix_len, page_size);
  ATLAS_REQUIRE(out_bytes >= sz.bytes, "out buffer holds %lld bytes, the spec needs %lld",
                static_cast<long long>(out_bytes), static_cast<long long>(sz.bytes));
  // 2. ancestor-or-self sets, nw words per node
  const int64_t nw = (n + 63) / 64;
  if (int64_t(sc.anc.size()) < n * nw) sc.anc.resize(n * nw);
  uint64_t* anc = sc.anc.data();
  for (int32_t i = 0; i < n; ++i) {
    uint64_t* a = anc + int64_t(i) * nw;
    if (parents_host[i] >= 0)
      std::memcpy(a, anc + int64_t(parents_host[i]) * nw, nw * sizeof(uint64_t));
    else
      std::memset(a, 0, nw * sizeof(uint64_t));
    a[i >> 6] |= uint64_t(1) << (i & 63);
  }
  // 3. [token ids | depths | mask words] (int64), [indptrs, last, page table] (int32), tree block (bytes)
  const int64_t kv_len = prefix_len + n;
  const int64_t pages = (kv_len + page_size - 1) / page_size;
  const int64_t last = kv_len - (pages - 1) * page_size;
  std::memcpy(out_host, sc.tok.data(), 8 * size_t(n));
  std::memcpy(out_host + 8 * n, sc.dep.data(), 8 * size_t(n));
  uint64_t* words = reinterpret_cast<uint64_t*>(out_host + 16 * n);
  if (n <= 64) {
    for (int32_t i = 0; i < n; ++i) words[i] = anc[i];
  } else if (sz.tiles) {
    // word j of node i: visibility of keys 64 * (prefix_len / 64 + j) + b,
    // prefix keys visible, tree key prefix_len + c iff c is an ancestor
    const int low = int(prefix_len & 63);
    for (int32_t i = 0; i < n; ++i) {
      const uint64_t* a = anc + int64_t(i) * nw;
      uint64_t* w = words + int64_t(i) * sz.tiles;
      for (int64_t j = 0; j < sz.tiles; ++j) {
        uint64_t v = j < nw ? a[j] << low : 0;
        if (low && j >= 1 && j - 1 < nw) v |= a[j - 1] >> (64 - low);
        if (j == 0 && low) v |= (uint64_t(1) << low) - 1;
        w[j] = v;
      }
    }
  }
  int32_t* i32 = reinterpret_cast<int32_t*>(out_host + 16 * n + 8 * sz.words);
  i32[0] = 0;
  i32[1] = n;
  i32[2] = 0;
  i32[3] = int32_t(pages);
  i32[4] = int32_t(last);
  for (int64_t p = 0; p < pages; ++p) i32[5 + p] = int32_t(p);
  for (int64_t p = 5 + pages; p < sz.i32_count; ++p) i32[p] = 0;
  uint8_t* block = out_host + 16 * n + 8 * sz.words + 4 * sz.i32_count;
  for (int32_t i = 0; i < n; ++i) {
    const uint64_t* a = anc + int64_t(i) * nw;
    uint8_t* row = block + int64_t(i) * n;
    for (int32_t j = 0; j < n; ++j) row[j] = uint8_t((a[j >> 6] >> (j & 63)) & 1);
  }
  info_host[0] = n;
  info_host[1] = kv_len;
  info_host[2] = pages;
  info_host[3] = last;
  info_host[4] = sz.words;
  info_host[5] = sz.tiles;
  info_host[6] = sz.i32_count;
  info_host[7] = sz.bytes;
  return ATLAS_OK;
}

namespace atlas {
namespace {

// Dense mask row i: keys below prefix_len visible, tree key prefix_len + j
// visible iff block[i][j]; four mask bytes per thread.
__global__ __launch_bounds__(256) void tree_mask_fill_kernel(const uint8_t* __restrict__ block, int32_t n,
                                                             int64_t prefix_len, uint8_t* __restrict__ mask,
                                                             int64_t total) {
  const int64_t kv_len = prefix_len + n;
  const int64_t f0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t f = f0 + b;
    if (f >= total) return;
    const int64_t row = f / kv_len;
    const int64_t col = f - row * kv_len;
    mask[f] = col < prefix_len ? uint8_t(1) : block[row * n + (col - prefix_len)];
  }
}

// The spec's bytes copied from src to dst by the first copy_blocks
// workgroups (16 bytes per thread), and the dense mask filled by the others
// from the tree block, the spec's last n * n bytes, read at src.  src may be
// mapped host memory: the launch then reads the spec once over the bus and
// no copy precedes it.
__global__ __launch_bounds__(256) void tree_spec_upload_kernel(const uint8_t* __restrict__ src, int64_t nbytes,
                                                               int32_t n, int64_t prefix_len,
                                                               uint8_t* __restrict__ dst,
                                                               uint8_t* __restrict__ mask, int64_t total,
                                                               int32_t copy_blocks) {
  if (int32_t(blockIdx.x) < copy_blocks) {
    const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 16;
    if (i + 16 <= nbytes) {
      *reinterpret_cast<uint4*>(dst + i) = *reinterpret_cast<const uint4*>(src + i);
    } else {
      for (int64_t b = i; b < nbytes; ++b) dst[b] = src[b];
    }
    return;
  }
  const uint8_t* block = src + (nbytes - int64_t(n) * n);
  const int64_t kv_len = prefix_len + n;
  const int64_t f0 = (int64_t(blockIdx.x - copy_blocks) * blockDim.x + threadIdx.x) * 4;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t f = f0 + b;
    if (f >= total) return;
    const int64_t row = f / kv_len;
    const int64_t col = f - row * kv_len;
    mask[f] = col < prefix_len ? uint8_t(1) : block[row * n + (col - prefix_len)];
  }
}

}  // namespace
}  // namespace atlas

extern "C" int atlas_tree_spec_upload(const uint8_t* spec_src, int64_t nbytes, int32_t n, int64_t prefix_len,
                                      uint8_t* spec_dev, uint8_t* mask_dev, void* stream) {
  ATLAS_REQUIRE(n > 0 && prefix_len >= 0, "n must be positive and prefix_len >= 0");
  ATLAS_REQUIRE(nbytes >= int64_t(n) * n, "the spec (%lld bytes) must end with its %d x %d tree block",
                static_cast<long long>(nbytes), n, n);
  ATLAS_REQUIRE(spec_src && spec_dev && mask_dev, "spec and mask buffers must not be NULL");
  ATLAS_REQUIRE(reinterpret_cast<uintptr_t>(spec_src) % 16 == 0 && reinterpret_cast<uintptr_t>(spec_dev) % 16 == 0,
                "spec buffers must be 16-byte aligned");
  const int64_t total = int64_t(n) * (prefix_len + n);
  const int64_t fill_blocks = ((total + 3) / 4 + 255) / 256;
  const int64_t copy_blocks = spec_src == spec_dev ? 0 : ((nbytes + 15) / 16 + 255) / 256;
  ATLAS_REQUIRE(fill_blocks + copy_blocks < (int64_t(1) << 31), "mask too large");
  hipLaunchKernelGGL(atlas::tree_spec_upload_kernel, dim3(unsigned(fill_blocks + copy_blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), spec_src, nbytes, n, prefix_len, spec_dev, mask_dev, total,
                     int32_t(copy_blocks));
  return atlas::launch_status("tree_spec_upload_kernel");
}

extern "C" int atlas_tree_mask_fill(const uint8_t* block_dev, int32_t n, int64_t prefix_len, uint8_t* mask_dev,
                                    void* stream) {
  ATLAS_REQUIRE(n > 0 && prefix_len >= 0, "n must be positive and prefix_len >= 0");
  ATLAS_REQUIRE(block_dev && mask_dev, "block and mask must not be NULL");
  const int64_t total = int64_t(n) * (prefix_len + n);
  const int64_t threads = (total + 3) / 4;
  ATLAS_REQUIRE(threads / 256 < (int64_t(1) << 31), "mask too large");
  hipLaunchKernelGGL(atlas::tree_mask_fill_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), block_dev, n, prefix_len, mask_dev, total);
  return atlas::launch_status("tree_mask_fill_kernel");
}
