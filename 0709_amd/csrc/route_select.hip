// Route selection of a Target verify on the device: the selected route and
// the commit positions of its nodes, computed from the scoring launch's
// log-probs in stream order, so the commit can be queued behind the scoring
// before the host has read the scores back.
//
// Follows target_runtime.py:567-573 (target_best: the maximum of
// (selection score, draft path log-prob, -route id); first_route),
// :722-765 (per-token log-probs rounded to the logits dtype, the route score
// as Python's left-to-right float sum, the weighted score), :754-760 (the
// fallback thresholds) and :873-920 (the commit positions).

#include "common.hpp"

namespace atlas {
namespace {

struct SelectArgs {
  const float* logprobs;
  int64_t* src;
  int64_t* dst;
  int32_t* result;
  float* host_out;  // mapped host memory for the values and the result, or NULL
  int64_t prefix_len;
  double path_threshold, first_threshold;
  int32_t num_routes, depth, policy, rounding, num_weights, has_path_threshold, has_first_threshold;
  double weights[ATLAS_SELECT_MAX_DEPTH];
  double draft_path[ATLAS_SELECT_MAX_ROUTES];
  int64_t route_id[ATLAS_SELECT_MAX_ROUTES];
  int32_t commit_len[ATLAS_SELECT_MAX_ROUTES];
  int16_t node[ATLAS_SELECT_MAX_ENTRIES];
};

// The fp32 log-prob as the host reads it after rounding to the logits dtype
// (round to nearest even; bf16 NaN becomes the canonical quiet NaN).
__device__ __forceinline__ float round_logits_dtype(float v, int rounding) {
  if (rounding == ATLAS_ROUND_F16) return static_cast<float>(static_cast<_Float16>(v));
  if (rounding == ATLAS_ROUND_BF16) {
    const uint32_t u = __float_as_uint(v);
    if (v != v) return __uint_as_float(0x7FC00000u);
    return __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
  }
  return v;
}

// Python's tuple comparison (a > b) of (score, draft, -id) keys: the first
// position whose values are not equal decides (NaN equals nothing).
__device__ __forceinline__ bool key_greater(double sa, double da, int64_t ia, double sb, double db, int64_t ib) {
  if (!(sa == sb)) return sa > sb;
  if (!(da == db)) return da > db;
  return ia < ib;
}

__global__ __launch_bounds__(64) void route_select_kernel(SelectArgs a) {
  // Python rounds every product and every sum: no fused multiply-adds.
#pragma clang fp contract(off)
  __shared__ double score[ATLAS_SELECT_MAX_ROUTES];
  __shared__ double first[ATLAS_SELECT_MAX_ROUTES];
  const int r = threadIdx.x;
  if (r < a.num_routes) {
    double target = 0.0, weighted = 0.0, f = 0.0;
    for (int t = 0; t < a.depth; ++t) {
      // scoring order: every route's first token, then each route's others
      const int idx = t == 0 ? r : a.num_routes + r * (a.depth - 1) + (t - 1);
      const double v = static_cast<double>(round_logits_dtype(a.logprobs[idx], a.rounding));
      if (t == 0) f = v;
      target = target + v;
      if (a.num_weights) weighted = weighted + a.weights[t] * v;
    }
    score[r] = a.num_weights ? weighted : target;
    first[r] = f;
  }
  __syncthreads();
  if (a.host_out != nullptr) {
    // the values as the host reads them (rounded to the logits dtype), with
    // the selection, so no separate copy follows
    const int n = a.num_routes * a.depth;
    for (int i = r; i < n; i += 64) a.host_out[i] = round_logits_dtype(a.logprobs[i], a.rounding);
  }
  if (r != 0) return;
  int best = 0;
  if (a.policy == ATLAS_SELECT_TARGET_BEST) {
    for (int i = 1; i < a.num_routes; ++i)
      if (key_greater(score[i], a.draft_path[i], a.route_id[i], score[best], a.draft_path[best], a.route_id[best]))
        best = i;
  }
  const bool fallback = (a.has_first_threshold && first[best] < a.first_threshold) ||
                        (a.has_path_threshold && score[best] < a.path_threshold);
  const int count = fallback ? 0 : a.commit_len[best];
  // rows past the committed count copy onto themselves (no change)
  for (int i = 0; i < a.depth; ++i) {
    const int64_t d = a.prefix_len + i;
    a.src[i] = i < count ? a.prefix_len + a.node[best * a.depth + i] : d;
    a.dst[i] = d;
  }
  a.result[0] = best;
  a.result[1] = count;
  if (a.host_out != nullptr) {
    int32_t* res = reinterpret_cast<int32_t*>(a.host_out + a.num_routes * a.depth);
    res[0] = best;
    res[1] = count;
  }
}

}  // namespace
}  // namespace atlas

extern "C" int atlas_route_select(const float* logprobs_dev, int num_routes, int depth, int policy, int rounding,
                                  const double* weights_host, int num_weights, const double* draft_path_host,
                                  const int64_t* route_ids_host, const int32_t* commit_len_host,
                                  const int32_t* node_ids_host, int has_path_threshold, double path_threshold,
                                  int has_first_threshold, double first_threshold, int64_t prefix_len,
                                  int64_t* src_dev, int64_t* dst_dev, int32_t* result_dev, float* host_out,
                                  void* stream) {
  ATLAS_REQUIRE(num_routes >= 1 && num_routes <= ATLAS_SELECT_MAX_ROUTES, "num_routes must be in [1, %d]",
                ATLAS_SELECT_MAX_ROUTES);
  ATLAS_REQUIRE(depth >= 1 && depth <= ATLAS_SELECT_MAX_DEPTH && num_routes * depth <= ATLAS_SELECT_MAX_ENTRIES,
                "depth must be in [1, %d] with num_routes * depth <= %d", ATLAS_SELECT_MAX_DEPTH,
                ATLAS_SELECT_MAX_ENTRIES);
  ATLAS_REQUIRE(policy == ATLAS_SELECT_TARGET_BEST || policy == ATLAS_SELECT_FIRST_ROUTE, "unknown policy %d",
                policy);
  ATLAS_REQUIRE(rounding == ATLAS_ROUND_NONE || rounding == ATLAS_ROUND_F16 || rounding == ATLAS_ROUND_BF16,
                "unknown rounding %d", rounding);
  ATLAS_REQUIRE(num_weights == 0 || num_weights == depth, "num_weights must be 0 or depth");
  ATLAS_REQUIRE(prefix_len >= 0, "prefix_len must be >= 0");
  ATLAS_REQUIRE(logprobs_dev && src_dev && dst_dev && result_dev && draft_path_host && route_ids_host &&
                    commit_len_host && node_ids_host && (weights_host || num_weights == 0),
                "buffers must not be NULL");
  atlas::SelectArgs a{};
  a.logprobs = logprobs_dev;
  a.src = src_dev;
  a.dst = dst_dev;
  a.result = result_dev;
  a.host_out = host_out;
  a.prefix_len = prefix_len;
  a.path_threshold = path_threshold;
  a.first_threshold = first_threshold;
  a.num_routes = num_routes;
  a.depth = depth;
  a.policy = policy;
  a.rounding = rounding;
  a.num_weights = num_weights;
  a.has_path_threshold = has_path_threshold ? 1 : 0;
  a.has_first_threshold = has_first_threshold ? 1 : 0;
  for (int t = 0; t < num_weights; ++t) a.weights[t] = weights_host[t];
  for (int r = 0; r < num_routes; ++r) {
    ATLAS_REQUIRE(commit_len_host[r] >= 0 && commit_len_host[r] <= depth, "route %d: commit length %d outside [0, %d]",
                  r, commit_len_host[r], depth);
    a.draft_path[r] = draft_path_host[r];
    a.route_id[r] = route_ids_host[r];
    a.commit_len[r] = commit_len_host[r];
    for (int t = 0; t < depth; ++t) {
      const int32_t n = node_ids_host[r * depth + t];
      ATLAS_REQUIRE(n >= 0 && n <= 32767, "route %d: node id %d outside [0, 32767]", r, n);
      a.node[r * depth + t] = static_cast<int16_t>(n);
    }
  }
  hipLaunchKernelGGL(atlas::route_select_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), a);
  return atlas::launch_status("route_select_kernel");
}
