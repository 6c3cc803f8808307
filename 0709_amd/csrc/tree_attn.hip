// Ancestor-masked paged tree / forest verify attention for gfx950.
//
// One workgroup (4 waves) handles one work item: a block of packed query rows
// (row = node * group + head_in_group, so the `group` query heads sharing a KV
// head are stacked as rows) of one KV head against one split of the request's
// keys.  Keys stream through LDS in tiles of 64 gathered through the page
// table; the next tile is prefetched into registers while the current one is
// multiplied.
//
// MFMA formulation (v_mfma_f32_16x16x32 f16/bf16), per 16-row tile:
//   S^T[key, row] = K[key, :] . Q[row, :]     A = K from LDS, B = Q in registers
//   O^T[dim, row] += V^T[dim, key] . P^T[key, row]
// The C layout of a 16x16 MFMA gives lane l the column l % 16 and rows
// 4*(l/16)..+3, so every lane holds scores and outputs of a single query row:
// the online softmax needs only two cross-lane reductions (max) per tile and
// none for the rescale.  P^T feeds the second MFMA straight from registers
// because V^T is written to LDS with its keys in the order in which the score
// tile's C layout hands them out (see vt_position).
//
// Masks are applied in registers: keys below mask_col_start are visible to
// every row, keys at and after it use the row's 64-bit ancestor bitmask; tiles
// wholly inside the always-visible range skip the mask code.
#include "common.hpp"

namespace atlas {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTileKeys = 64;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const char* q;
  int64_t q_stride_token;  // elements
  int64_t q_stride_head;   // elements
  const char* kv;
  int64_t page_stride;  // bytes
  int64_t v_offset;     // bytes
  int64_t token_stride; // bytes
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* kv_len;
  const uint64_t* tree_mask;
  const int32_t* mask_col_start;
  const atlas_attn_work_t* work;
  char* out;
  int64_t out_stride_token;  // elements
  int64_t out_stride_head;   // elements
  float* lse;
  float* part_o;
  float* part_lse;
  float scale_log2;  // sm_scale * log2(e)
  int mask_mode;
  int group;
  int num_qo_heads;
  int page_size;
  int page_shift;
};

template <bool BF16>
struct Mfma;

template <>
struct Mfma<false> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    _Float16 h = static_cast<_Float16>(x);
    return __builtin_bit_cast(uint16_t, h);
  }
};

template <>
struct Mfma<true> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    __bf16 h = static_cast<__bf16>(x);
    return __builtin_bit_cast(uint16_t, h);
  }
};

// Position inside a 32-key block of V^T at which key k (0..31) is stored.  The
// B operand of the P.V MFMA is built from two score tiles: lane group g holds
// keys 4g..4g+3 of the first tile and 16+4g..16+4g+3 of the second as its
// eight k-elements 8g..8g+7, so V^T stores key k at that same k-element.
__device__ __forceinline__ int vt_position(int k) {
  return ((k & 15) >> 2) * 8 + ((k >> 4) << 2) + (k & 3);
}

__device__ __forceinline__ float wave_max_across_groups(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ float wave_sum_across_groups(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

template <int D, bool BF16, int RT>
__global__ __launch_bounds__(kThreads) void tree_attn_kernel(AttnArgs a) {
  typedef Mfma<BF16> M;
  typedef typename M::frag frag;
  constexpr int KS = D / 32;           // k-steps of the score MFMA
  constexpr int DT = D / 16;           // 16-dim output tiles
  constexpr int CH = D / 8;            // 16-byte chunks per key row
  constexpr int KROW = D + 8;          // K row stride in LDS (elements)
  constexpr int VROW = kTileKeys + 8;  // V^T row stride in LDS (elements)
  constexpr int NKV = kTileKeys * CH / kThreads;  // K vectors per thread
  constexpr int KPT = NKV;                        // keys per thread for V (same count)
  static_assert(NKV == 2 || NKV == 4, "head_dim must be 64 or 128");

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kTileKeys * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[D * VROW];

  const atlas_attn_work_t w = a.work[blockIdx.x];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = lane >> 4;
  const int r16 = lane & 15;

  const int req = w.req;
  const int kvh = w.kv_head;
  const int qo_start = a.qo_indptr[req];
  const int qo_len = a.qo_indptr[req + 1] - qo_start;
  const int kv_len = a.kv_len[req];
  const int pt_base = a.kv_indptr[req];
  const int kv_end = min(w.kv_end, kv_len);
  const int G = a.group;
  const int64_t head_off = int64_t(kvh) * D * 2;

  // Mask window: keys < vis_all are visible to every row.
  int vis_all = kv_end;
  int col0 = 0;
  if (a.mask_mode == ATLAS_MASK_TREE) {
    col0 = a.mask_col_start[req];
    vis_all = min(vis_all, col0);
  } else if (a.mask_mode == ATLAS_MASK_CAUSAL) {
    vis_all = min(vis_all, kv_len - qo_len + 1);
  }

  frag qf[RT][KS];
  f32x4 o[RT][DT];
  float m_run[RT];
  float l_run[RT];
  uint64_t tbits[RT];
  int climit[RT];
  int node_of[RT];
  int head_of[RT];
  bool row_ok[RT];

#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int lr = (wave + kWaves * rt) * 16 + r16;
    row_ok[rt] = lr < w.num_rows;
    const int prow = w.row_start + lr;
    node_of[rt] = prow / G;
    head_of[rt] = kvh * G + (prow - node_of[rt] * G);
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.f;
    tbits[rt] = 0;
    climit[rt] = 0;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (row_ok[rt]) {
      const char* qrow = a.q + ((int64_t(qo_start + node_of[rt]) * a.q_stride_token +
                                 int64_t(head_of[rt]) * a.q_stride_head) * 2);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint4 v = *reinterpret_cast<const uint4*>(qrow + (ks * 32 + grp * 8) * 2);
        qf[rt][ks] = __builtin_bit_cast(frag, v);
      }
      if (a.mask_mode == ATLAS_MASK_TREE) tbits[rt] = a.tree_mask[qo_start + node_of[rt]];
      if (a.mask_mode == ATLAS_MASK_CAUSAL) climit[rt] = kv_len - qo_len + node_of[rt];
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[rt][ks] = __builtin_bit_cast(frag, uint4{0, 0, 0, 0});
    }
  }

  // Global -> register staging of one key tile.
  uint4 kreg[NKV];
  uint4 vreg[KPT];
  const int v_chunk = tid % CH;
  const int v_key0 = (tid / CH) * KPT;

  auto key_addr = [&](int p) -> const char* {
    const int lp = a.page_shift >= 0 ? (p >> a.page_shift) : (p / a.page_size);
    const int off = p - lp * a.page_size;
    const int64_t page = a.kv_indices[pt_base + lp];
    return a.kv + page * a.page_stride + int64_t(off) * a.token_stride + head_off;
  };

  auto load_tile = [&](int t0) {
#pragma unroll
    for (int j = 0; j < NKV; ++j) {
      const int v = tid + kThreads * j;
      const int kk = v / CH;
      const int c = v % CH;
      const int p = t0 + kk;
      kreg[j] = uint4{0, 0, 0, 0};
      if (p < kv_end) kreg[j] = *reinterpret_cast<const uint4*>(key_addr(p) + c * 16);
    }
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int p = t0 + v_key0 + j;
      vreg[j] = uint4{0, 0, 0, 0};
      if (p < kv_end)
        vreg[j] = *reinterpret_cast<const uint4*>(key_addr(p) + a.v_offset + v_chunk * 16);
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < NKV; ++j) {
      const int v = tid + kThreads * j;
      const int kk = v / CH;
      const int c = v % CH;
      *reinterpret_cast<uint4*>(&k_lds[kk * KROW + c * 8]) = kreg[j];
    }
    // Transpose KPT keys x 8 dims into 8 dim rows of KPT keys.
    const int pos = (v_key0 >> 5) * 32 + vt_position(v_key0 & 31);
    const uint16_t* e[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) e[j] = reinterpret_cast<const uint16_t*>(&vreg[j]);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      uint16_t* dst = &vt_lds[(v_chunk * 8 + d) * VROW + pos];
      if constexpr (KPT == 4) {
        const uint32_t lo = uint32_t(e[0][d]) | (uint32_t(e[1][d]) << 16);
        const uint32_t hi = uint32_t(e[2][d]) | (uint32_t(e[3][d]) << 16);
        *reinterpret_cast<uint2*>(dst) = uint2{lo, hi};
      } else {
        *reinterpret_cast<uint32_t*>(dst) = uint32_t(e[0][d]) | (uint32_t(e[1][d]) << 16);
      }
    }
  };

  int t0 = w.kv_start;
  if (t0 < kv_end) load_tile(t0);

  for (; t0 < kv_end; t0 += kTileKeys) {
    __syncthreads();  // previous tile's LDS reads are done
    store_tile();
    __syncthreads();
    if (t0 + kTileKeys < kv_end) load_tile(t0 + kTileKeys);

    // ---- scores S^T = K Q^T ----
    f32x4 s[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[rt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint4 av = *reinterpret_cast<const uint4*>(&k_lds[(kt * 16 + r16) * KROW + ks * 32 + grp * 8]);
        const frag af = __builtin_bit_cast(frag, av);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          if ((wave + kWaves * rt) * 16 < w.num_rows) s[rt][kt] = M::run(af, qf[rt][ks], s[rt][kt]);
        }
      }
    }

    // ---- online softmax, P^T fragments ----
    const bool need_mask = (t0 + kTileKeys) > vis_all;
    frag pf[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if ((wave + kWaves * rt) * 16 >= w.num_rows) {
        pf[rt][0] = pf[rt][1] = __builtin_bit_cast(frag, uint4{0, 0, 0, 0});
        continue;
      }
      float x[4][4];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = s[rt][kt][i] * a.scale_log2;
          if (need_mask) {
            const int p = t0 + kt * 16 + grp * 4 + i;
            bool vis = p < kv_end;
            if (vis && p >= vis_all) {
              if (a.mask_mode == ATLAS_MASK_TREE) {
                const int b = p - col0;
                vis = b < 64 && ((tbits[rt] >> b) & 1ull);
              } else if (a.mask_mode == ATLAS_MASK_CAUSAL) {
                vis = p <= climit[rt];
              }
            }
            v = vis ? v : -INFINITY;
          }
          x[kt][i] = v;
          mx = fmaxf(mx, v);
        }
      }
      mx = wave_max_across_groups(mx);
      const float m_new = fmaxf(m_run[rt], mx);
      const bool dead = m_new == -INFINITY;
      const float alpha = dead ? 1.f : __builtin_amdgcn_exp2f(m_run[rt] - m_new);
      float psum = 0.f;
      uint16_t ph[4][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pe = dead ? 0.f : __builtin_amdgcn_exp2f(x[kt][i] - m_new);
          psum += pe;
          ph[kt][i] = M::from_float(pe);
        }
      }
      l_run[rt] = l_run[rt] * alpha + psum;
      m_run[rt] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[rt][dt] *= alpha;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        u16x8 u;
        u[0] = ph[2 * kk][0];
        u[1] = ph[2 * kk][1];
        u[2] = ph[2 * kk][2];
        u[3] = ph[2 * kk][3];
        u[4] = ph[2 * kk + 1][0];
        u[5] = ph[2 * kk + 1][1];
        u[6] = ph[2 * kk + 1][2];
        u[7] = ph[2 * kk + 1][3];
        pf[rt][kk] = __builtin_bit_cast(frag, u);
      }
    }

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const uint4 av = *reinterpret_cast<const uint4*>(&vt_lds[(dt * 16 + r16) * VROW + kk * 32 + grp * 8]);
        const frag af = __builtin_bit_cast(frag, av);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          if ((wave + kWaves * rt) * 16 < w.num_rows) o[rt][dt] = M::run(af, pf[rt][kk], o[rt][dt]);
        }
      }
    }
  }

  // ---- epilogue ----
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if ((wave + kWaves * rt) * 16 >= w.num_rows) continue;
    const float l_tot = wave_sum_across_groups(l_run[rt]);
    if (!row_ok[rt]) continue;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const float lse2 = l_tot > 0.f ? m_run[rt] + __builtin_log2f(l_tot) : -INFINITY;
    const int lr = (wave + kWaves * rt) * 16 + r16;
    if (w.partial_row < 0) {
      char* orow = a.out + ((int64_t(qo_start + node_of[rt]) * a.out_stride_token +
                             int64_t(head_of[rt]) * a.out_stride_head) * 2);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint32_t lo = uint32_t(M::from_float(o[rt][dt][0] * inv)) |
                            (uint32_t(M::from_float(o[rt][dt][1] * inv)) << 16);
        const uint32_t hi = uint32_t(M::from_float(o[rt][dt][2] * inv)) |
                            (uint32_t(M::from_float(o[rt][dt][3] * inv)) << 16);
        *reinterpret_cast<uint2*>(orow + (dt * 16 + grp * 4) * 2) = uint2{lo, hi};
      }
      if (a.lse != nullptr && grp == 0)
        a.lse[int64_t(qo_start + node_of[rt]) * a.num_qo_heads + head_of[rt]] = lse2 * kLn2;
    } else {
      const int64_t prow = int64_t(w.partial_row) + lr;
      float* po = a.part_o + prow * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f32x4 v = o[rt][dt] * inv;
        *reinterpret_cast<f32x4*>(po + dt * 16 + grp * 4) = v;
      }
      if (grp == 0) a.part_lse[prow] = lse2;
    }
  }
}

struct MergeArgs {
  const atlas_attn_merge_t* merge;
  const int32_t* qo_indptr;
  const float* part_o;
  const float* part_lse;
  char* out;
  int64_t out_stride_token;
  int64_t out_stride_head;
  float* lse;
  int group;
  int num_qo_heads;
};

// One wave per packed row: combine the row's split states.
template <int D, bool BF16>
__global__ __launch_bounds__(256) void tree_attn_merge_kernel(MergeArgs a) {
  typedef Mfma<BF16> M;
  constexpr int PER = D / 64;
  const atlas_attn_merge_t mi = a.merge[blockIdx.x];
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (row >= mi.num_rows) return;
  float mx = -INFINITY;
  for (int s = 0; s < mi.num_splits; ++s)
    mx = fmaxf(mx, a.part_lse[int64_t(mi.partial_row) + int64_t(s) * mi.num_rows + row]);
  float acc[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) acc[i] = 0.f;
  float wsum = 0.f;
  if (mx != -INFINITY) {
    for (int s = 0; s < mi.num_splits; ++s) {
      const int64_t prow = int64_t(mi.partial_row) + int64_t(s) * mi.num_rows + row;
      const float ws = __builtin_amdgcn_exp2f(a.part_lse[prow] - mx);
      wsum += ws;
      const float* po = a.part_o + prow * D + lane * PER;
#pragma unroll
      for (int i = 0; i < PER; ++i) acc[i] += ws * po[i];
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const int prow_q = mi.row_start + row;
  const int node = prow_q / a.group;
  const int head = mi.kv_head * a.group + (prow_q - node * a.group);
  const int qo_start = a.qo_indptr[mi.req];
  uint16_t* orow = reinterpret_cast<uint16_t*>(
      a.out + ((int64_t(qo_start + node) * a.out_stride_token + int64_t(head) * a.out_stride_head) * 2));
#pragma unroll
  for (int i = 0; i < PER; ++i) orow[lane * PER + i] = M::from_float(acc[i] * inv);
  if (a.lse != nullptr && lane == 0)
    a.lse[int64_t(qo_start + node) * a.num_qo_heads + head] =
        wsum > 0.f ? (mx + __builtin_log2f(wsum)) * kLn2 : -INFINITY;
}

template <int D, bool BF16>
int launch_attn(const AttnArgs& args, int num_work, int rt, const MergeArgs& margs, int num_merge,
                int max_rows, hipStream_t stream) {
  int rc;
  switch (rt) {
    case 1:
      hipLaunchKernelGGL((tree_attn_kernel<D, BF16, 1>), dim3(num_work), dim3(kThreads), 0, stream, args);
      break;
    case 2:
      hipLaunchKernelGGL((tree_attn_kernel<D, BF16, 2>), dim3(num_work), dim3(kThreads), 0, stream, args);
      break;
    case 3:
      hipLaunchKernelGGL((tree_attn_kernel<D, BF16, 3>), dim3(num_work), dim3(kThreads), 0, stream, args);
      break;
    default:
      set_error("unsupported row tiles per wave %d", rt);
      return ATLAS_EUNSUPPORTED;
  }
  if ((rc = launch_status("tree_attn_kernel"))) return rc;
  if (num_merge > 0) {
    const dim3 grid(num_merge, (max_rows + 3) / 4);
    hipLaunchKernelGGL((tree_attn_merge_kernel<D, BF16>), grid, dim3(256), 0, stream, margs);
    if ((rc = launch_status("tree_attn_merge_kernel"))) return rc;
  }
  return ATLAS_OK;
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" int atlas_tree_verify_attn(
    const void* q, int64_t q_stride_token, int64_t q_stride_head, const void* kv_cache,
    int64_t page_stride, int64_t kv_v_offset, int64_t token_stride, const int32_t* qo_indptr_dev,
    const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev, const int32_t* kv_len_dev,
    int mask_mode, const uint64_t* tree_mask_dev, const int32_t* mask_col_start_dev,
    const atlas_attn_work_t* work_dev, int num_work, const atlas_attn_merge_t* merge_dev,
    int num_merge, int max_rows_per_item, int num_qo_heads, int num_kv_heads, int head_dim,
    int page_size, float sm_scale, int dtype, void* out, int64_t out_stride_token,
    int64_t out_stride_head, float* lse, void* workspace_dev, size_t workspace_bytes,
    void* stream) {
  ATLAS_REQUIRE(q && kv_cache && out, "q, kv_cache and out must not be NULL");
  ATLAS_REQUIRE(qo_indptr_dev && kv_indptr_dev && kv_indices_dev && kv_len_dev,
                "indptr / indices / kv_len arrays must not be NULL");
  ATLAS_REQUIRE(num_qo_heads > 0 && num_kv_heads > 0 && num_qo_heads % num_kv_heads == 0,
                "num_qo_heads must be a positive multiple of num_kv_heads");
  ATLAS_REQUIRE(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128, got %d", head_dim);
  ATLAS_REQUIRE(page_size > 0, "page_size must be positive");
  ATLAS_REQUIRE(dtype == ATLAS_DTYPE_F16 || dtype == ATLAS_DTYPE_BF16, "dtype must be f16 or bf16");
  ATLAS_REQUIRE(mask_mode >= ATLAS_MASK_NONE && mask_mode <= ATLAS_MASK_CAUSAL, "bad mask mode %d",
                mask_mode);
  ATLAS_REQUIRE(mask_mode != ATLAS_MASK_TREE || (tree_mask_dev && mask_col_start_dev),
                "tree mask mode needs tree_mask and mask_col_start");
  ATLAS_REQUIRE(num_work >= 0 && num_merge >= 0, "negative work counts");
  ATLAS_REQUIRE(max_rows_per_item > 0 && max_rows_per_item <= 3 * kWaves * 16,
                "max_rows_per_item %d out of range (1..%d)", max_rows_per_item, 3 * kWaves * 16);
  ATLAS_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15) == 0 && (reinterpret_cast<uintptr_t>(kv_cache) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & 7) == 0,
                "q / kv_cache must be 16-byte aligned and out 8-byte aligned");
  ATLAS_REQUIRE(q_stride_head % 8 == 0 && q_stride_token % 8 == 0 && out_stride_head % 4 == 0 &&
                    out_stride_token % 4 == 0,
                "q strides must be multiples of 8 elements and out strides multiples of 4");
  ATLAS_REQUIRE(page_stride % 16 == 0 && token_stride % 16 == 0 && kv_v_offset % 16 == 0,
                "kv strides must be multiples of 16 bytes");
  if (num_work == 0) return ATLAS_OK;
  ATLAS_REQUIRE(work_dev != nullptr, "work list must not be NULL");
  const int row_tiles = (max_rows_per_item + 15) / 16;
  const int rt = (row_tiles + kWaves - 1) / kWaves;
  ATLAS_REQUIRE(rt >= 1 && rt <= 3, "rows per item %d exceeds %d", max_rows_per_item, 3 * kWaves * 16);

  AttnArgs args{};
  args.q = static_cast<const char*>(q);
  args.q_stride_token = q_stride_token;
  args.q_stride_head = q_stride_head;
  args.kv = static_cast<const char*>(kv_cache);
  args.page_stride = page_stride;
  args.v_offset = kv_v_offset;
  args.token_stride = token_stride;
  args.qo_indptr = qo_indptr_dev;
  args.kv_indptr = kv_indptr_dev;
  args.kv_indices = kv_indices_dev;
  args.kv_len = kv_len_dev;
  args.tree_mask = tree_mask_dev;
  args.mask_col_start = mask_col_start_dev;
  args.work = work_dev;
  args.out = static_cast<char*>(out);
  args.out_stride_token = out_stride_token;
  args.out_stride_head = out_stride_head;
  args.lse = lse;
  args.scale_log2 = sm_scale * kLog2e;
  args.mask_mode = mask_mode;
  args.group = num_qo_heads / num_kv_heads;
  args.num_qo_heads = num_qo_heads;
  args.page_size = page_size;
  args.page_shift = ilog2_exact(page_size);

  MergeArgs margs{};
  if (num_merge > 0) {
    ATLAS_REQUIRE(merge_dev != nullptr && workspace_dev != nullptr, "split work needs merge list and workspace");
    // The planner places the partial O rows first and the partial LSE after
    // them: workspace = [partial_rows * D floats][partial_rows floats].
    ATLAS_REQUIRE(workspace_bytes % (size_t(head_dim + 1) * 4) == 0,
                  "workspace_bytes must be partial_rows * (head_dim + 1) * 4");
    const size_t partial_rows = workspace_bytes / (size_t(head_dim + 1) * 4);
    args.part_o = static_cast<float*>(workspace_dev);
    args.part_lse = args.part_o + partial_rows * head_dim;
    margs.merge = merge_dev;
    margs.qo_indptr = qo_indptr_dev;
    margs.part_o = args.part_o;
    margs.part_lse = args.part_lse;
    margs.out = args.out;
    margs.out_stride_token = out_stride_token;
    margs.out_stride_head = out_stride_head;
    margs.lse = lse;
    margs.group = args.group;
    margs.num_qo_heads = num_qo_heads;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == ATLAS_DTYPE_BF16;
  if (head_dim == 128)
    return bf16 ? launch_attn<128, true>(args, num_work, rt, margs, num_merge, max_rows_per_item, s)
                : launch_attn<128, false>(args, num_work, rt, margs, num_merge, max_rows_per_item, s);
  return bf16 ? launch_attn<64, true>(args, num_work, rt, margs, num_merge, max_rows_per_item, s)
              : launch_attn<64, false>(args, num_work, rt, margs, num_merge, max_rows_per_item, s);
}
