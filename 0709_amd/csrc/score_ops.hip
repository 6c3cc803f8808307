// Route scoring: per-row log-sum-exp over the vocabulary and the gather of the
// log-probabilities of the verified tokens, so a verify needs one small
// device-to-host copy instead of one scalar read per token.
#include "common.hpp"

namespace atlas {
namespace {

constexpr int kThreads = 1024;

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

__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(v, off);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red[] reuse across calls
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) t = is_max ? fmaxf(t, red[w]) : t + red[w];
  return t;
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

// Block r: log-sum-exp of logits row r (natural log, fp32) in two passes over
// the row -- the maximum, then the sum of exp2((x - max) * log2 e) (the second
// pass reads the row back from L2) -- with 16-byte loads when the row is
// 16-byte aligned; then every gather that reads row r.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void gather_logprobs_kernel(const char* logits, int64_t row_stride_bytes,
                                                                   int64_t vocab, const int32_t* rows,
                                                                   const int64_t* tokens, int64_t n,
                                                                   float* row_lse, float* out) {
  __shared__ float red[kThreads / 64];
  __shared__ float lse_sh;
  constexpr float kLog2e = 1.4426950408889634f;
  constexpr int EPV = Vec<DT>::kElems;
  const int r = blockIdx.x;
  const char* row = logits + int64_t(r) * row_stride_bytes;
  const int64_t nvec = VEC ? vocab / EPV : 0;

  float m = -INFINITY;
  for (int64_t v = threadIdx.x; v < nvec; v += kThreads) {
    Vec<DT> x;
    x.load(row + v * 16);
#pragma unroll
    for (int k = 0; k < EPV; ++k) m = fmaxf(m, x.x[k]);
  }
  for (int64_t i = nvec * EPV + threadIdx.x; i < vocab; i += kThreads) m = fmaxf(m, load_logit<DT>(row, i));
  m = block_reduce(m, true, red);

  const float mb = m == -INFINITY ? 0.f : m * kLog2e;
  float s = 0.f;
  for (int64_t v = threadIdx.x; v < nvec; v += kThreads) {
    Vec<DT> x;
    x.load(row + v * 16);
#pragma unroll
    for (int k = 0; k < EPV; ++k) s += __builtin_amdgcn_exp2f(__builtin_fmaf(x.x[k], kLog2e, -mb));
  }
  for (int64_t i = nvec * EPV + threadIdx.x; i < vocab; i += kThreads)
    s += __builtin_amdgcn_exp2f(__builtin_fmaf(load_logit<DT>(row, i), kLog2e, -mb));
  s = block_reduce(s, false, red);

  if (threadIdx.x == 0) {
    lse_sh = m + logf(s);
    if (row_lse) row_lse[r] = lse_sh;
  }
  __syncthreads();
  const float lse = lse_sh;
  for (int64_t i = threadIdx.x; i < n; i += kThreads) {
    if (rows[i] != r) continue;
    const int64_t t = tokens[i];
    out[i] = (t >= 0 && t < vocab) ? load_logit<DT>(row, t) - lse : NAN;
  }
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" int atlas_gather_logprobs(const void* logits_dev, int64_t row_stride, int64_t num_rows, int64_t vocab,
                                     int dtype, const int32_t* row_dev, const int64_t* token_dev, int64_t n,
                                     float* row_lse_dev, float* out_dev, void* stream) {
  ATLAS_REQUIRE(logits_dev && num_rows > 0 && vocab > 0, "bad logits arguments");
  ATLAS_REQUIRE(n == 0 || (row_dev && token_dev && out_dev), "gather buffers must not be NULL");
  ATLAS_REQUIRE(num_rows < (int64_t(1) << 31), "too many rows");
  const int es = dtype == ATLAS_DTYPE_F32 ? 4 : 2;
  ATLAS_REQUIRE(dtype == ATLAS_DTYPE_F32 || dtype == ATLAS_DTYPE_F16 || dtype == ATLAS_DTYPE_BF16, "bad dtype");
  ATLAS_REQUIRE(row_stride >= vocab, "row_stride (elements) must cover the vocabulary");
  const int64_t stride_bytes = row_stride * es;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* lg = static_cast<const char*>(logits_dev);
  const dim3 grid(static_cast<unsigned>(num_rows));
  const bool vec = (reinterpret_cast<uintptr_t>(logits_dev) % 16) == 0 && stride_bytes % 16 == 0;
#define ATLAS_GATHER_LAUNCH(DT)                                                                              \
  do {                                                                                                       \
    if (vec)                                                                                                 \
      hipLaunchKernelGGL((gather_logprobs_kernel<DT, true>), grid, dim3(kThreads), 0, s, lg, stride_bytes,   \
                         vocab, row_dev, token_dev, n, row_lse_dev, out_dev);                                \
    else                                                                                                     \
      hipLaunchKernelGGL((gather_logprobs_kernel<DT, false>), grid, dim3(kThreads), 0, s, lg, stride_bytes,  \
                         vocab, row_dev, token_dev, n, row_lse_dev, out_dev);                                \
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
