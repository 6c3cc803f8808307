// Route scoring: per-row log-sum-exp over the vocabulary and the gather of the
// log-probabilities of the verified tokens, so a verify needs one small
// device-to-host copy instead of one scalar read per token.
#include <algorithm>

#include "common.hpp"

namespace atlas {
namespace {

constexpr int kThreads = 256;

template <int DT>
__device__ __forceinline__ float load_logit(const char* row, int64_t i) {
  if constexpr (DT == ATLAS_DTYPE_F32) {
    return reinterpret_cast<const float*>(row)[i];
  } else if constexpr (DT == ATLAS_DTYPE_F16) {
    return static_cast<float>(reinterpret_cast<const _Float16*>(row)[i]);
  } else {
    return static_cast<float>(reinterpret_cast<const __bf16*>(row)[i]);
  }
}

// 16 bytes of logits -> up to 8 floats.
template <int DT>
struct Vec {
  static constexpr int kElems = DT == ATLAS_DTYPE_F32 ? 4 : 8;
  float x[kElems];
  __device__ __forceinline__ void load(const char* p) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    if constexpr (DT == ATLAS_DTYPE_F32) {
      x[0] = __uint_as_float(u.x);
      x[1] = __uint_as_float(u.y);
      x[2] = __uint_as_float(u.z);
      x[3] = __uint_as_float(u.w);
    } else {
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (DT == ATLAS_DTYPE_F16) {
          x[2 * k] = static_cast<float>(__builtin_bit_cast(_Float16, uint16_t(w[k] & 0xffff)));
          x[2 * k + 1] = static_cast<float>(__builtin_bit_cast(_Float16, uint16_t(w[k] >> 16)));
        } else {
          x[2 * k] = __uint_as_float(w[k] << 16);
          x[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
        }
      }
    }
  }
};

// Workgroup (c, r) reads chunk c of logits row r once: the chunk's maximum m
// and the sum of exp(x - m), kept online per thread (16-byte loads when the
// rows are 16-byte aligned), then reduced over the workgroup.  It stores the
// pair into its slot of the row and counts itself in on the row's arrival
// counter with one agent-scope read-modify-write that releases the slot; the
// workgroup that arrives last (the counter held num_chunks - 1) acquires
// every slot, combines the pairs in chunk order (a fixed order, so the LSE is
// the same on every run), writes the row LSE and every gather of row r, and
// empties the slots and the counter for the next call.  A slot is
// (max bits, ~sum bits); every slot is written before its workgroup arrives.
struct GatherArgs {
  const char* logits;
  int64_t row_stride_bytes;
  const char* logits2;          // rows num_rows1 .. come from here (or null)
  int64_t row_stride2_bytes;
  int64_t num_rows1;
  int64_t vocab;
  const int32_t* rows;
  const int64_t* tokens;
  int64_t n;
  float* row_lse;
  float* out;
  uint64_t* slots;     // [num_rows, num_chunks], zero between calls
  uint32_t* arrivals;  // [num_rows], zero between calls
  int num_chunks;
  int64_t chunk_len;  // elements, a multiple of 8 (the last chunk may be shorter)
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kPre = 2;  // gathers per thread whose logits are loaded ahead of the combine

// (m, s) pairs: s is a sum of exp(x - m).
__device__ __forceinline__ void pair_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = s * __builtin_amdgcn_exp2f((m - mn) * kLog2e) + s2 * __builtin_amdgcn_exp2f((m2 - mn) * kLog2e);
  m = mn;
}

template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void gather_logprobs_kernel(GatherArgs a) {
  __shared__ float red_m[kThreads / 64];
  __shared__ float red_s[kThreads / 64];
  __shared__ int last_sh;
  __shared__ float lse_sh;
  constexpr int EPV = Vec<DT>::kElems;
  const int c = blockIdx.x;
  const int r = blockIdx.y;
  const int t = threadIdx.x;
  const char* row = r < a.num_rows1 ? a.logits + int64_t(r) * a.row_stride_bytes
                                    : a.logits2 + (int64_t(r) - a.num_rows1) * a.row_stride2_bytes;
  const int64_t c0 = int64_t(c) * a.chunk_len;
  const int64_t c1 = min(a.vocab, c0 + a.chunk_len);

  // Row and token of the first kPre * kThreads gathers, requested before the
  // chunk (no branch on them: a branch would wait for them first).
  int32_t grow[kPre];
  int64_t gtok[kPre];
#pragma unroll
  for (int k = 0; k < kPre; ++k) {
    const int64_t i = min(t + int64_t(k) * kThreads, max(a.n - 1, int64_t(0)));
    grow[k] = a.n > 0 ? a.rows[i] : -1;
    gtok[k] = a.n > 0 ? a.tokens[i] : 0;
  }

  float m = -INFINITY, s = 0.f;
  int64_t scalar0 = c0;
  if constexpr (VEC) {
    // whole vectors of the chunk (chunk starts are multiples of 8 elements)
    const int64_t v0 = c0 / EPV;
    const int64_t v1 = c1 / EPV;
    scalar0 = v1 * EPV;
#pragma unroll 4
    for (int64_t v = v0 + t; v < v1; v += kThreads) {
      Vec<DT> x;
      x.load(row + v * 16);
      float vm = x.x[0];
#pragma unroll
      for (int k = 1; k < EPV; ++k) vm = fmaxf(vm, x.x[k]);
      const float mn = fmaxf(m, vm);
      float acc = m == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f((m - mn) * kLog2e);
      const float mb = mn == -INFINITY ? 0.f : mn * kLog2e;  // (an all -inf vector adds zeros)
#pragma unroll
      for (int k = 0; k < EPV; ++k) acc += __builtin_amdgcn_exp2f(__builtin_fmaf(x.x[k], kLog2e, -mb));
      m = mn;
      s = acc;
    }
  }
  for (int64_t i = scalar0 + t; i < c1; i += kThreads) {
    const float x = load_logit<DT>(row, i);
    pair_merge(m, s, x, 1.f);
  }
  // The gathered logits go out now and land while the pair is published.
  float gx[kPre];
  bool gmine[kPre];
#pragma unroll
  for (int k = 0; k < kPre; ++k) {
    gmine[k] = t + int64_t(k) * kThreads < a.n && grow[k] == r;
    const bool ok = gtok[k] >= 0 && gtok[k] < a.vocab;
    gx[k] = load_logit<DT>(row, ok ? gtok[k] : 0);
    if (!ok) gx[k] = NAN;
  }
  // workgroup reduction of (m, s)
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) pair_merge(m, s, __shfl_xor(m, off), __shfl_xor(s, off));
  if ((t & 63) == 0) {
    red_m[t >> 6] = m;
    red_s[t >> 6] = s;
  }
  __syncthreads();
  uint64_t* rs = a.slots + int64_t(r) * a.num_chunks;
  if (t == 0) {
    float bm = red_m[0], bs = red_s[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) pair_merge(bm, bs, red_m[w], red_s[w]);
    const uint64_t slot = uint64_t(__float_as_uint(bm)) | (uint64_t(~__float_as_uint(bs)) << 32);
    __hip_atomic_store(rs + c, slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // The release orders the slot before the arrival; the last arriver's
    // acquire then sees every slot (all earlier arrivals released theirs).
    const uint32_t prev = __hip_atomic_fetch_add(a.arrivals + r, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == uint32_t(a.num_chunks - 1);
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    last_sh = last;
  }
  __syncthreads();
  if (!last_sh) return;

  // The last arriver: combine the row's slots in chunk order (one per lane of
  // wave 0, then a fixed pairwise tree).
  if (t < 64) {
    float cm = -INFINITY, cs = 0.f;
    for (int k = t; k < a.num_chunks; k += 64) {
      const uint64_t v = __hip_atomic_load(rs + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pair_merge(cm, cs, __uint_as_float(uint32_t(v)), __uint_as_float(~uint32_t(v >> 32)));
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) pair_merge(cm, cs, __shfl_xor(cm, off), __shfl_xor(cs, off));
    if (t == 0) lse_sh = cm + __builtin_log2f(cs) * kLn2;
  }
  __syncthreads();
  const float lse = lse_sh;
  if (t == 0) {
    if (a.row_lse) a.row_lse[r] = lse;
    __hip_atomic_store(a.arrivals + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  for (int k = t; k < a.num_chunks; k += kThreads)
    __hip_atomic_store(rs + k, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int k = 0; k < kPre; ++k)
    if (gmine[k]) a.out[t + int64_t(k) * kThreads] = gx[k] - lse;
  for (int64_t i = t + int64_t(kPre) * kThreads; i < a.n; i += kThreads) {
    if (a.rows[i] != r) continue;
    const int64_t tok = a.tokens[i];
    a.out[i] = (tok >= 0 && tok < a.vocab) ? load_logit<DT>(row, tok) - lse : NAN;
  }
}

}  // namespace
}  // namespace atlas

using namespace atlas;

namespace atlas {
namespace {
// Chunks per row: about ATLAS_GATHER_TARGET_WGS (row, chunk) workgroups in
// all, chunks of at least 1024 logits, at most 256 chunks per row.  Every
// workgroup ends with an agent-scope release (the L2 write-back that orders
// its slot before its arrival), so fewer, longer chunks win: 35 rows x 128256
// fp16 logits take 8.4 us with 128 workgroups, 9.0 with 256 and 10.4 with 512
// (9.3 with 64 and 12.4 with one workgroup per row).
struct GatherGeom {
  int num_chunks;
  int64_t chunk_len;
};
#ifndef ATLAS_GATHER_TARGET_WGS
#define ATLAS_GATHER_TARGET_WGS 128
#endif
GatherGeom gather_geom(int64_t num_rows, int64_t vocab) {
  const int64_t want = (ATLAS_GATHER_TARGET_WGS + num_rows - 1) / num_rows;
  const int64_t by_len = (vocab + 1023) / 1024;
  int64_t chunks = std::max<int64_t>(1, std::min<int64_t>({want, by_len, 256}));
  int64_t len = (vocab + chunks - 1) / chunks;
  len = (len + 7) / 8 * 8;
  chunks = (vocab + len - 1) / len;
  return GatherGeom{int(chunks), len};
}
}  // namespace
}  // namespace atlas

extern "C" int64_t atlas_gather_logprobs_workspace_bytes(int64_t num_rows, int64_t vocab) {
  if (num_rows <= 0 || vocab <= 0 || num_rows >= (int64_t(1) << 31)) return -1;
  const GatherGeom g = gather_geom(num_rows, vocab);
  // the slots, then one arrival counter per row
  return int64_t(size_t(num_rows) * g.num_chunks * sizeof(uint64_t) + size_t(num_rows) * sizeof(uint32_t));
}

extern "C" int atlas_gather_logprobs(const void* logits_dev, int64_t row_stride, int64_t num_rows,
                                     const void* logits2_dev, int64_t row_stride2, int64_t num_rows2, int64_t vocab,
                                     int dtype, const int32_t* row_dev, const int64_t* token_dev, int64_t n,
                                     float* row_lse_dev, float* out_dev, void* workspace_dev, size_t workspace_bytes,
                                     void* stream) {
  ATLAS_REQUIRE(logits_dev && num_rows > 0 && vocab > 0, "bad logits arguments");
  ATLAS_REQUIRE(num_rows2 >= 0 && (num_rows2 == 0 || logits2_dev != nullptr), "bad second logits arguments");
  ATLAS_REQUIRE(n == 0 || (row_dev && token_dev && out_dev), "gather buffers must not be NULL");
  const int64_t total_rows = num_rows + num_rows2;
  ATLAS_REQUIRE(total_rows < (int64_t(1) << 31), "too many rows");
  const int es = dtype == ATLAS_DTYPE_F32 ? 4 : 2;
  ATLAS_REQUIRE(dtype == ATLAS_DTYPE_F32 || dtype == ATLAS_DTYPE_F16 || dtype == ATLAS_DTYPE_BF16, "bad dtype");
  ATLAS_REQUIRE(row_stride >= vocab && (num_rows2 == 0 || row_stride2 >= vocab),
                "row strides (elements) must cover the vocabulary");
  const int64_t need = atlas_gather_logprobs_workspace_bytes(total_rows, vocab);
  ATLAS_REQUIRE(workspace_dev != nullptr && workspace_bytes >= size_t(need),
                "workspace of %lld bytes needed (atlas_gather_logprobs_workspace_bytes), got %zu", (long long)need,
                workspace_bytes);
  ATLAS_REQUIRE((reinterpret_cast<uintptr_t>(workspace_dev) & 15) == 0, "workspace must be 16-byte aligned");
  const GatherGeom g = gather_geom(total_rows, vocab);
  GatherArgs a{};
  a.logits = static_cast<const char*>(logits_dev);
  a.row_stride_bytes = row_stride * es;
  a.logits2 = static_cast<const char*>(logits2_dev);
  a.row_stride2_bytes = row_stride2 * es;
  a.num_rows1 = num_rows;
  a.vocab = vocab;
  a.rows = row_dev;
  a.tokens = token_dev;
  a.n = n;
  a.row_lse = row_lse_dev;
  a.out = out_dev;
  a.slots = static_cast<uint64_t*>(workspace_dev);
  a.arrivals = reinterpret_cast<uint32_t*>(a.slots + total_rows * g.num_chunks);
  a.num_chunks = g.num_chunks;
  a.chunk_len = g.chunk_len;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(g.num_chunks), static_cast<unsigned>(total_rows));
  const bool vec = (reinterpret_cast<uintptr_t>(logits_dev) % 16) == 0 && a.row_stride_bytes % 16 == 0 &&
                   (num_rows2 == 0 ||
                    ((reinterpret_cast<uintptr_t>(logits2_dev) % 16) == 0 && a.row_stride2_bytes % 16 == 0));
#define ATLAS_GATHER_LAUNCH(DT)                                                                          \
  do {                                                                                                   \
    if (vec)                                                                                             \
      hipLaunchKernelGGL((gather_logprobs_kernel<DT, true>), grid, dim3(kThreads), 0, s, a);             \
    else                                                                                                 \
      hipLaunchKernelGGL((gather_logprobs_kernel<DT, false>), grid, dim3(kThreads), 0, s, a);            \
  } while (0)
  if (dtype == ATLAS_DTYPE_F32)
    ATLAS_GATHER_LAUNCH(ATLAS_DTYPE_F32);
  else if (dtype == ATLAS_DTYPE_F16)
    ATLAS_GATHER_LAUNCH(ATLAS_DTYPE_F16);
  else
    ATLAS_GATHER_LAUNCH(ATLAS_DTYPE_BF16);
#undef ATLAS_GATHER_LAUNCH
  return launch_status("gather_logprobs_kernel");
}
