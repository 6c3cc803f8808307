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

// Block r: lse of logits row r (natural log, fp32 accumulation), then every
// gather that reads row r.
template <int DT>
__global__ __launch_bounds__(kThreads) void gather_logprobs_kernel(const char* logits, int64_t row_stride_bytes,
                                                                   int64_t vocab, const int32_t* rows,
                                                                   const int64_t* tokens, int64_t n,
                                                                   float* row_lse, float* out) {
  __shared__ float red_m[kThreads / 64];
  __shared__ float red_s[kThreads / 64];
  const int r = blockIdx.x;
  const char* row = logits + int64_t(r) * row_stride_bytes;
  float m = -INFINITY, s = 0.f;
  for (int64_t i = threadIdx.x; i < vocab; i += kThreads) {
    const float x = load_logit<DT>(row, i);
    if (x > m) {
      s = s * expf(m - x) + 1.f;
      m = x;
    } else {
      s += expf(x - m);
    }
  }
  // Wave reduction of (m, s) pairs.
  for (int off = 32; off > 0; off >>= 1) {
    const float om = __shfl_xor(m, off);
    const float os = __shfl_xor(s, off);
    const float nm = fmaxf(m, om);
    const float a = (m == -INFINITY) ? 0.f : s * expf(m - nm);
    const float b = (om == -INFINITY) ? 0.f : os * expf(om - nm);
    m = nm;
    s = a + b;
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red_m[wave] = m;
    red_s[wave] = s;
  }
  __syncthreads();
  __shared__ float lse_sh;
  if (threadIdx.x == 0) {
    float mm = -INFINITY, ss = 0.f;
    for (int w = 0; w < kThreads / 64; ++w) {
      const float nm = fmaxf(mm, red_m[w]);
      const float a = (mm == -INFINITY) ? 0.f : ss * expf(mm - nm);
      const float b = (red_m[w] == -INFINITY) ? 0.f : red_s[w] * expf(red_m[w] - nm);
      mm = nm;
      ss = a + b;
    }
    lse_sh = mm + logf(ss);
    if (row_lse) row_lse[r] = lse_sh;
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < n; i += kThreads) {
    if (rows[i] != r) continue;
    const int64_t t = tokens[i];
    out[i] = (t >= 0 && t < vocab) ? load_logit<DT>(row, t) - lse_sh : NAN;
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
  if (dtype == ATLAS_DTYPE_F32)
    hipLaunchKernelGGL(gather_logprobs_kernel<ATLAS_DTYPE_F32>, grid, dim3(kThreads), 0, s, lg, stride_bytes, vocab,
                       row_dev, token_dev, n, row_lse_dev, out_dev);
  else if (dtype == ATLAS_DTYPE_F16)
    hipLaunchKernelGGL(gather_logprobs_kernel<ATLAS_DTYPE_F16>, grid, dim3(kThreads), 0, s, lg, stride_bytes, vocab,
                       row_dev, token_dev, n, row_lse_dev, out_dev);
  else
    hipLaunchKernelGGL(gather_logprobs_kernel<ATLAS_DTYPE_BF16>, grid, dim3(kThreads), 0, s, lg, stride_bytes, vocab,
                       row_dev, token_dev, n, row_lse_dev, out_dev);
  return launch_status("gather_logprobs_kernel");
}
