// Shared internals of the gfx950 paged-KV library: error reporting, vector
// types and the per-launch layer table carried in the kernel argument block.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/atlas0709.h"

namespace atlas {

// Message of the last failing call on this thread (atlas_last_error()).
void set_error(const char* fmt, ...);

// Translate a HIP status into the ABI's error convention.
inline int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return ATLAS_OK;
  set_error("%s: %s", what, hipGetErrorString(err));
  return ATLAS_EHIP_BASE - static_cast<int>(err);
}

// Check the launch that was just enqueued.
inline int launch_status(const char* what) { return hip_status(hipGetLastError(), what); }

#define ATLAS_REQUIRE(cond, ...)     \
  do {                               \
    if (!(cond)) {                   \
      ::atlas::set_error(__VA_ARGS__); \
      return ATLAS_EINVAL;           \
    }                                \
  } while (0)

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Per-launch layer base addresses (K and V), carried by value so a launch
// needs no device-side pointer table.
struct LayerTable {
  const char* k[ATLAS_MAX_LAYERS_PER_LAUNCH];
  const char* v[ATLAS_MAX_LAYERS_PER_LAUNCH];
};

// Physical slot -> byte offset inside one layer's K (or V) region.
struct SlotGeom {
  int64_t page_stride;
  int64_t token_stride;
  int64_t page_size;
  int32_t page_shift;  // log2(page_size) when a power of two, else -1
  int32_t row_vecs;    // 16-byte vectors per token row
  int32_t row_shift;   // log2(row_vecs) when a power of two, else -1
  int32_t head_shift;  // rows split by KV head (HND pages): log2(16-byte vectors per head), else -1
  int64_t head_stride; // bytes between a token's KV heads when head_shift >= 0
};

__device__ __forceinline__ int64_t slot_offset(int64_t slot, const SlotGeom& g) {
  int64_t page, off;
  if (g.page_shift >= 0) {
    page = slot >> g.page_shift;
    off = slot & (g.page_size - 1);
  } else {
    page = slot / g.page_size;
    off = slot - page * g.page_size;
  }
  return page * g.page_stride + off * g.token_stride;
}

// Byte offset of 16-byte vector `vec` of a token row from the row's first
// byte: contiguous rows (NHD pages, flat pools), or one run of vectors per KV
// head, head_stride apart (HND pages).
__device__ __forceinline__ int64_t vec_offset(int vec, const SlotGeom& g) {
  if (g.head_shift < 0) return int64_t(vec) * 16;
  return int64_t(vec >> g.head_shift) * g.head_stride + int64_t(vec & ((1 << g.head_shift) - 1)) * 16;
}

__device__ __forceinline__ void split_row(int64_t idx, const SlotGeom& g, int64_t& item, int& vec) {
  if (g.row_shift >= 0) {
    item = idx >> g.row_shift;
    vec = static_cast<int>(idx & (g.row_vecs - 1));
  } else {
    item = idx / g.row_vecs;
    vec = static_cast<int>(idx - item * g.row_vecs);
  }
}

inline int ilog2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

}  // namespace atlas
