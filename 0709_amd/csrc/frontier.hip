// Drafter frontier: the top-k next tokens of every parent row by log-softmax
// probability, the candidates they make, and the stable multi-key order /
// selection of those candidates, written in the int64 record layout the host
// materialises with one copy.
//
// A frontier step is two launches over a (chunk, row) grid:
//   frontier_stats_kernel  per chunk: maximum and sum of exp(x - max);
//   frontier_topk_kernel   per chunk: the row's log-sum-exp from the chunk
//                          statistics, then the chunk's k best keys.  The last
//                          chunk of a row to finish merges the row's lists and
//                          writes its candidates; the last row to finish orders
//                          and selects all candidates (last-arriver counters,
//                          cleared by the stats launch; no workgroup waits
//                          for another).
// The ordering works on any candidate batch as its own launch too
// (candidate_select_kernel).
#include "common.hpp"

namespace atlas {
namespace {

constexpr int kFThreads = 256;
constexpr int kMaxK = ATLAS_MAX_FRONTIER_K;
constexpr int kMaxCand = ATLAS_MAX_FRONTIER_CANDIDATES;
constexpr int kMaxChunks = kFThreads;  // the row merge gives each chunk list one thread
constexpr int kTile = 512;             // candidates per LDS tile of the ordering

// ---------------------------------------------------------------- keys
// Order-preserving map of a float to u32 (larger float -> larger key).
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// A token's key: the value, then the smaller token id on equal values.  Real
// keys are never 0 (ids are below 2^31), so 0 marks an empty slot.
__device__ __forceinline__ uint64_t token_key(float v, uint32_t id) {
  return (uint64_t(fkey(v)) << 32) | uint64_t(0xffffffffu - id);
}
__device__ __forceinline__ uint32_t key_id(uint64_t k) { return 0xffffffffu - uint32_t(k); }
__device__ __forceinline__ float key_value(uint64_t k) { return fkey_inv(uint32_t(k >> 32)); }

template <int DT>
__device__ __forceinline__ float round_dt(float x) {
  if constexpr (DT == ATLAS_DTYPE_F16) return static_cast<float>(static_cast<_Float16>(x));
  else if constexpr (DT == ATLAS_DTYPE_BF16) return static_cast<float>(static_cast<__bf16>(x));
  else return x;
}

template <int DT>
__device__ __forceinline__ float load_one(const char* row, int64_t i) {
  if constexpr (DT == ATLAS_DTYPE_F32) return reinterpret_cast<const float*>(row)[i];
  else if constexpr (DT == ATLAS_DTYPE_F16) return static_cast<float>(reinterpret_cast<const _Float16*>(row)[i]);
  else return static_cast<float>(reinterpret_cast<const __bf16*>(row)[i]);
}

// 16 aligned bytes of a row -> 8 (16-bit types) or 4 (fp32) floats.
template <int DT>
struct Group {
  static constexpr int kElems = DT == ATLAS_DTYPE_F32 ? 4 : 8;
  float x[kElems];
  __device__ __forceinline__ void load(const char* p) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == ATLAS_DTYPE_F32) {
        x[k] = __uint_as_float(w[k]);
      } else if constexpr (DT == ATLAS_DTYPE_F16) {
        x[2 * k] = static_cast<float>(__builtin_bit_cast(_Float16, uint16_t(w[k] & 0xffffu)));
        x[2 * k + 1] = static_cast<float>(__builtin_bit_cast(_Float16, uint16_t(w[k] >> 16)));
      } else {
        x[2 * k] = __uint_as_float(w[k] << 16);
        x[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      }
    }
  }
};

// Visits x[i] for i in [c0, c1) of a row: 16-byte groups when the row is
// 16-byte aligned (c0 is a multiple of 8 elements), single loads otherwise.
template <int DT, typename F>
__device__ __forceinline__ void for_chunk(const char* row, int64_t c0, int64_t c1, F&& f) {
  constexpr int E = Group<DT>::kElems;
  const int t = threadIdx.x;
  int64_t i0 = c0;
  if ((reinterpret_cast<uintptr_t>(row) & 15) == 0) {
    const int64_t ng = (c1 - c0) / E;
    for (int64_t g = t; g < ng; g += kFThreads) {
      Group<DT> v;
      v.load(row + (c0 + g * E) * (DT == ATLAS_DTYPE_F32 ? 4 : 2));
#pragma unroll
      for (int k = 0; k < E; ++k) f(c0 + g * E + k, v.x[k]);
    }
    i0 = c0 + ng * E;
  }
  for (int64_t i = i0 + t; i < c1; i += kFThreads) f(i, load_one<DT>(row, i));
}

// ---------------------------------------------------------------- reductions
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<int>(uint32_t(v)), m);
  const uint32_t hi = __shfl_xor(static_cast<int>(uint32_t(v >> 32)), m);
  return (uint64_t(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const uint64_t o = shfl_xor_u64(v, m);
    v = o > v ? o : v;
  }
  return v;
}

// Online (max, sum of exp(x - max)) pairs.
__device__ __forceinline__ void ms_add(float& m, float& s, float m2, float s2) {
  if (m2 == -INFINITY) return;
  if (m == -INFINITY) {
    m = m2;
    s = s2;
    return;
  }
  if (m2 > m) {
    s = s * expf(m - m2) + s2;
    m = m2;
  } else {
    s = s + s2 * expf(m2 - m);
  }
}

// Block combine of per-thread (m, s) in a fixed order (waves by xor steps,
// then wave 0..3), so every workgroup of a row derives the same result.
__device__ __forceinline__ void block_ms(float& m, float& s, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o);
    const float s2 = __shfl_xor(s, o);
    ms_add(m, s, m2, s2);
  }
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    red[2 * wave] = m;
    red[2 * wave + 1] = s;
  }
  __syncthreads();
  m = red[0];
  s = red[1];
#pragma unroll
  for (int w = 1; w < kFThreads / 64; ++w) ms_add(m, s, red[2 * w], red[2 * w + 1]);
}

// A thread's KM best keys, descending (0 = empty); `thr` is entry k - 1.
template <int KM>
struct TopList {
  uint64_t a[KM];
  uint64_t thr;
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int i = 0; i < KM; ++i) a[i] = 0;
    thr = 0;
  }
  __device__ __forceinline__ void push(uint64_t key, int k) {
    if (key <= thr) return;
#pragma unroll
    for (int i = 0; i < KM; ++i) {
      const bool sw = key > a[i];
      const uint64_t old = a[i];
      a[i] = sw ? key : old;
      key = sw ? old : key;
    }
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < KM; ++i) t = (i == k - 1) ? a[i] : t;
    thr = t;
  }
};

// The k largest keys held by the block's threads (each list sorted, keys
// distinct) -> out[0..k), descending.  Each wave merges its 64 lists by k
// rounds of wave maxima, then wave 0 merges the four wave lists the same way.
template <int KM>
__device__ __forceinline__ void block_topk(const TopList<KM>& L, int k, uint64_t* lists, uint64_t* wave_lists,
                                           uint64_t* out) {
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
#pragma unroll
  for (int i = 0; i < KM; ++i)
    if (i < k) lists[t * KM + i] = L.a[i];
  __syncthreads();
  int p = 0;
  uint64_t head = lists[t * KM];
  for (int r = 0; r < k; ++r) {
    const uint64_t m = wave_max_u64(head);
    if (head == m && m != 0) {
      ++p;
      head = p < k ? lists[t * KM + p] : 0;
    }
    if (lane == 0) wave_lists[wave * KM + r] = m;
  }
  __syncthreads();
  if (wave == 0) {
    p = 0;
    head = lane < kFThreads / 64 ? wave_lists[lane * KM] : 0;
    for (int r = 0; r < k; ++r) {
      const uint64_t m = wave_max_u64(head);
      if (lane < kFThreads / 64 && head == m && m != 0) {
        ++p;
        head = p < k ? wave_lists[lane * KM + p] : 0;
      }
      if (lane == 0) out[r] = m;
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- ordering
// Candidate columns (element strides), as the host's candidate tensors hold them.
struct CandCols {
  const int64_t* parent;
  const int64_t* root;
  const int64_t* token;
  const int64_t* rank;
  const double* cum;
  const double* plp;
  int64_t s_parent, s_root, s_token, s_rank, s_cum, s_plp;
};

// Descending order of doubles as u64: NaN first (torch sorts NaN above every
// number), -0.0 equal to +0.0.
__device__ __forceinline__ uint64_t dorder(double x) {
  if (x != x) return ~0ull;
  if (x == 0.0) x = 0.0;
  const uint64_t u = __double_as_longlong(x);
  return (u >> 63) ? ~u : (u | (1ull << 63));
}

struct Cand {
  int64_t root;
  uint64_t cum;  // dorder(cumulative log-prob)
  int64_t parent;
  int64_t rank;
  int64_t token;
};

__device__ __forceinline__ Cand load_cand(const CandCols& c, int64_t i) {
  Cand r;
  r.root = c.root[i * c.s_root];
  r.cum = dorder(c.cum[i * c.s_cum]);
  r.parent = c.parent[i * c.s_parent];
  r.rank = c.rank[i * c.s_rank];
  r.token = c.token[i * c.s_token];
  return r;
}

// Does candidate a (index ia) come before b (index ib)?  Keys: stage-1 root
// ascending (by_root), cumulative log-prob descending, parent route, rank in
// parent, token id ascending, then the original index (a stable sort's order).
__device__ __forceinline__ bool cand_before(const Cand& a, int64_t ia, const Cand& b, int64_t ib, bool by_root) {
  if (by_root && a.root != b.root) return a.root < b.root;
  if (a.cum != b.cum) return a.cum > b.cum;
  if (a.parent != b.parent) return a.parent < b.parent;
  if (a.rank != b.rank) return a.rank < b.rank;
  if (a.token != b.token) return a.token < b.token;
  return ia < ib;
}

struct SelectSmem {
  Cand tile[kTile];
  int pos[kMaxCand];  // position in the order (per root: inside the candidate's root)
  int sel[kMaxCand];  // selection order, or -1
};

enum SelectMode : int {
  kOrder = ATLAS_FRONTIER_ORDER,
  kOrderByRoot = ATLAS_FRONTIER_ORDER_BY_ROOT,
  kSelectGlobal = ATLAS_FRONTIER_SELECT_GLOBAL,
  kSelectPerRoot = ATLAS_FRONTIER_SELECT_PER_ROOT,
  kPack = ATLAS_FRONTIER_PACK,
};

struct SelectArgs {
  CandCols cols;
  int64_t count;
  int mode;
  int64_t num_selected;        // top-n (global / per root)
  const int64_t* selected_in;  // kPack: the selection, in order
  int64_t num_selected_in;
  const int64_t* node_ids;     // extra records of kind 1, or null
  int64_t num_node_ids;
  int64_t* order_out;     // kOrder / kOrderByRoot: position -> candidate
  int64_t* selected_out;  // kSelect*: selection order -> candidate
  int64_t* records;       // [count + num_node_ids, 8] or null
  bool records_filled;    // columns 0..6 already hold the candidates
};

// Position of every candidate in the order: the number of candidates that come
// before it (per root: before it inside its root), counted against LDS tiles
// of the candidates.  One workgroup of kFThreads.
__device__ void count_before(const SelectArgs& a, SelectSmem& sm, bool by_root, bool within_root) {
  const int t = threadIdx.x;
  const int64_t C = a.count;
  for (int64_t base = 0; base < C; base += kFThreads) {
    const int64_t c = base + t;
    const bool mine = c < C;
    Cand me{};
    if (mine) me = load_cand(a.cols, c);
    int before = 0;
    for (int64_t t0 = 0; t0 < C; t0 += kTile) {
      const int n = static_cast<int>(min<int64_t>(kTile, C - t0));
      __syncthreads();
      for (int j = t; j < n; j += kFThreads) sm.tile[j] = load_cand(a.cols, t0 + j);
      __syncthreads();
      if (mine)
        for (int j = 0; j < n; ++j) {
          const Cand& x = sm.tile[j];
          const bool b = cand_before(x, t0 + j, me, c, by_root) && (!within_root || x.root == me.root);
          before += b ? 1 : 0;
        }
    }
    if (mine) sm.pos[c] = before;
  }
  __syncthreads();
}

__device__ void select_block(const SelectArgs& a, SelectSmem& sm) {
  const int t = threadIdx.x;
  const int64_t C = a.count;
  switch (a.mode) {
    case kOrder:
    case kOrderByRoot:
      count_before(a, sm, a.mode == kOrderByRoot, false);
      for (int64_t c = t; c < C; c += kFThreads) a.order_out[sm.pos[c]] = c;
      return;
    case kSelectGlobal:
      count_before(a, sm, false, false);
      for (int64_t c = t; c < C; c += kFThreads) {
        const int p = sm.pos[c];
        const bool chosen = p < a.num_selected;
        sm.sel[c] = chosen ? p : -1;
        if (chosen) a.selected_out[p] = c;
      }
      break;
    case kSelectPerRoot:
      count_before(a, sm, true, true);
      // selection offset of a root = the selected candidates of lower roots
      for (int64_t base = 0; base < C; base += kFThreads) {
        const int64_t c = base + t;
        const bool mine = c < C;
        const int64_t my_root = mine ? a.cols.root[c * a.cols.s_root] : 0;
        int off = 0;
        for (int64_t t0 = 0; t0 < C; t0 += kTile) {
          const int n = static_cast<int>(min<int64_t>(kTile, C - t0));
          __syncthreads();
          for (int j = t; j < n; j += kFThreads) sm.tile[j].root = a.cols.root[(t0 + j) * a.cols.s_root];
          __syncthreads();
          if (mine)
            for (int j = 0; j < n; ++j) off += (sm.tile[j].root < my_root && sm.pos[t0 + j] < a.num_selected) ? 1 : 0;
        }
        if (mine) {
          const int in_root = sm.pos[c];
          const bool chosen = in_root < a.num_selected;
          sm.sel[c] = chosen ? off + in_root : -1;
          if (chosen) a.selected_out[off + in_root] = c;
        }
      }
      break;
    default:  // kPack
      for (int64_t c = t; c < C; c += kFThreads) sm.sel[c] = -1;
      __syncthreads();
      if (t == 0)
        for (int64_t i = 0; i < a.num_selected_in; ++i) {
          const int64_t c = a.selected_in[i];
          if (c >= 0 && c < C) sm.sel[c] = static_cast<int>(i);
        }
      break;
  }
  __syncthreads();
  if (a.records == nullptr) return;
  for (int64_t c = t; c < C; c += kFThreads) {
    int64_t* r = a.records + c * 8;
    if (!a.records_filled) {
      r[0] = 0;
      r[1] = a.cols.parent[c * a.cols.s_parent];
      r[2] = a.cols.root[c * a.cols.s_root];
      r[3] = a.cols.token[c * a.cols.s_token];
      r[4] = a.cols.rank[c * a.cols.s_rank];
      r[5] = __double_as_longlong(a.cols.cum[c * a.cols.s_cum]);
      r[6] = __double_as_longlong(a.cols.plp[c * a.cols.s_plp]);
    }
    r[7] = sm.sel[c];
  }
  for (int64_t i = t; i < a.num_node_ids; i += kFThreads) {
    int64_t* r = a.records + (C + i) * 8;
    r[0] = 1;
    r[1] = a.node_ids[i];
#pragma unroll
    for (int j = 2; j < 8; ++j) r[j] = 0;
  }
}

__global__ __launch_bounds__(kFThreads) void candidate_select_kernel(SelectArgs a) {
  __shared__ SelectSmem sm;
  select_block(a, sm);
}

// ---------------------------------------------------------------- top-k
struct FrontierArgs {
  const char* logits;
  int64_t row_stride_bytes;
  int64_t vocab;
  const float* proposal;  // Gumbel proposal scores [rows, vocab] (fp32), or null
  int64_t proposal_stride;
  int rows, k, num_chunks;
  int64_t chunk_len;
  const int64_t* parent_info;  // [rows, 3]: route id, stage-1 root id, log-prob bits
  void* token_logprobs;        // [rows, k] in the logits dtype
  int64_t* token_ids;          // [rows, k]
  int64_t* parent_rows;        // [rows * k] or null
  int32_t* counters;           // rows + 1 last-arriver counters (cleared by the stats launch)
  float2* stats;               // [rows, num_chunks]
  uint64_t* lists;             // [rows, num_chunks, k]
  SelectArgs sel;              // mode < 0: no records / selection
};

template <int DT>
__global__ __launch_bounds__(kFThreads) void frontier_stats_kernel(FrontierArgs a) {
  __shared__ float red[2 * kFThreads / 64];
  const int chunk = blockIdx.x;
  const int row = blockIdx.y;
  // The top-k launch's last-arriver counters start from zero: this launch
  // ends before that one starts.
  if (chunk == 0 && threadIdx.x == 0) {
    a.counters[row] = 0;
    if (row == 0) a.counters[a.rows] = 0;
  }
  const char* rp = a.logits + int64_t(row) * a.row_stride_bytes;
  const int64_t c0 = int64_t(chunk) * a.chunk_len;
  const int64_t c1 = min(a.vocab, c0 + a.chunk_len);
  float m = -INFINITY, s = 0.f;
  for_chunk<DT>(rp, c0, c1, [&](int64_t, float x) {
    if (x > m) {
      s = (m == -INFINITY ? 0.f : s * expf(m - x)) + 1.f;
      m = x;
    } else if (x != -INFINITY) {
      s += expf(x - m);
    }
  });
  block_ms(m, s, red);
  if (threadIdx.x == 0) a.stats[int64_t(row) * a.num_chunks + chunk] = float2{m, s};
}

template <int DT, int KM>
__global__ __launch_bounds__(kFThreads) void frontier_topk_kernel(FrontierArgs a) {
  // The top-k lists and the ordering's tiles are never live together.
  struct TopSmem {
    uint64_t lists[kFThreads * KM];
    uint64_t wave_lists[(kFThreads / 64) * KM];
    uint64_t best[KM];
  };
  __shared__ float red[2 * kFThreads / 64];
  __shared__ int flag;
  __shared__ __attribute__((aligned(16))) char smem[sizeof(TopSmem) > sizeof(SelectSmem) ? sizeof(TopSmem)
                                                                                          : sizeof(SelectSmem)];
  TopSmem& ts = *reinterpret_cast<TopSmem*>(smem);
  SelectSmem& sm = *reinterpret_cast<SelectSmem*>(smem);
  uint64_t* const lists = ts.lists;
  uint64_t* const wave_lists = ts.wave_lists;
  uint64_t* const best = ts.best;
  const int t = threadIdx.x;
  const int chunk = blockIdx.x;
  const int row = blockIdx.y;
  const int k = a.k;
  const char* rp = a.logits + int64_t(row) * a.row_stride_bytes;

  // The row's log-sum-exp from its chunk statistics (same order everywhere).
  float m = -INFINITY, s = 0.f;
  if (t < a.num_chunks) {
    const float2 st = a.stats[int64_t(row) * a.num_chunks + t];
    m = st.x;
    s = st.y;
  }
  block_ms(m, s, red);
  const float row_max = m;
  const float lse = logf(s);

  const int64_t c0 = int64_t(chunk) * a.chunk_len;
  const int64_t c1 = min(a.vocab, c0 + a.chunk_len);
  TopList<KM> L;
  L.clear();
  if (a.proposal == nullptr) {
    // log_softmax rounded to the logits dtype: ((x - max) - lse)
    for_chunk<DT>(rp, c0, c1, [&](int64_t i, float x) {
      L.push(token_key(round_dt<DT>((x - row_max) - lse), uint32_t(i)), k);
    });
  } else {
    const char* pp = reinterpret_cast<const char*>(a.proposal + int64_t(row) * a.proposal_stride);
    for_chunk<ATLAS_DTYPE_F32>(pp, c0, c1, [&](int64_t i, float x) { L.push(token_key(x, uint32_t(i)), k); });
  }
  block_topk<KM>(L, k, lists, wave_lists, best);
  uint64_t* my_list = a.lists + (int64_t(row) * a.num_chunks + chunk) * k;
  if (t < k) my_list[t] = best[t];

  // Last chunk of the row merges the row.
  __threadfence();
  __syncthreads();
  if (t == 0) flag = atomicAdd(&a.counters[row], 1) == a.num_chunks - 1;
  __syncthreads();
  if (!flag) return;
  __threadfence();
  L.clear();
  if (t < a.num_chunks) {
    const uint64_t* src = a.lists + (int64_t(row) * a.num_chunks + t) * k;
#pragma unroll
    for (int i = 0; i < KM; ++i)
      if (i < k) L.a[i] = src[i];
  }
  block_topk<KM>(L, k, lists, wave_lists, best);
  if (t < k) {
    const uint64_t key = best[t];
    const uint32_t id = key_id(key);
    float lp;
    if (a.proposal == nullptr) lp = key_value(key);
    else lp = round_dt<DT>((load_one<DT>(rp, id) - row_max) - lse);
    const int64_t c = int64_t(row) * k + t;
    if constexpr (DT == ATLAS_DTYPE_F32) {
      reinterpret_cast<float*>(a.token_logprobs)[c] = lp;
    } else if constexpr (DT == ATLAS_DTYPE_F16) {
      reinterpret_cast<_Float16*>(a.token_logprobs)[c] = static_cast<_Float16>(lp);
    } else {
      reinterpret_cast<__bf16*>(a.token_logprobs)[c] = static_cast<__bf16>(lp);
    }
    a.token_ids[c] = id;
    if (a.parent_rows != nullptr) a.parent_rows[c] = row;
    if (a.sel.records != nullptr) {
      int64_t* r = a.sel.records + c * 8;
      const int64_t* pi = a.parent_info + int64_t(row) * 3;
      const double plp = __longlong_as_double(pi[2]);
      r[0] = 0;
      r[1] = pi[0];
      r[2] = pi[1];
      r[3] = id;
      r[4] = t;
      r[5] = __double_as_longlong(plp + static_cast<double>(lp));
      r[6] = pi[2];
      r[7] = -1;
    }
  }
  if (a.sel.mode < 0) return;

  // Last row orders and selects every candidate (best[] is read above before
  // the barrier that precedes the ordering's first use of the shared bytes).
  __threadfence();
  __syncthreads();
  if (t == 0) flag = atomicAdd(&a.counters[a.rows], 1) == a.rows - 1;
  __syncthreads();
  if (!flag) return;
  __threadfence();
  select_block(a.sel, sm);
}

template <int DT, int KM>
int launch_topk(const FrontierArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((frontier_topk_kernel<DT, KM>), grid, dim3(kFThreads), 0, s, a);
  return launch_status("frontier_topk_kernel");
}

template <int DT>
int launch_frontier(const FrontierArgs& a, hipStream_t s) {
  const dim3 grid(a.num_chunks, a.rows);
  hipLaunchKernelGGL((frontier_stats_kernel<DT>), grid, dim3(kFThreads), 0, s, a);
  int rc = launch_status("frontier_stats_kernel");
  if (rc != ATLAS_OK) return rc;
  if (a.k <= 4) return launch_topk<DT, 4>(a, grid, s);
  if (a.k <= 8) return launch_topk<DT, 8>(a, grid, s);
  if (a.k <= 16) return launch_topk<DT, 16>(a, grid, s);
  return launch_topk<DT, 32>(a, grid, s);
}

struct Geometry {
  int num_chunks;
  int64_t chunk_len;
};

// Chunks of a multiple of 8 elements, enough (row, chunk) workgroups to cover
// the device about twice, at most kMaxChunks per row.
Geometry frontier_geometry(int64_t rows, int64_t vocab) {
  constexpr int64_t kTargetGroups = 1024;
  int64_t nc = (kTargetGroups + rows - 1) / rows;
  nc = std::min<int64_t>(nc, (vocab + 1023) / 1024);
  nc = std::max<int64_t>(1, std::min<int64_t>(nc, kMaxChunks));
  int64_t len = (vocab + nc - 1) / nc;
  len = (len + 7) / 8 * 8;
  nc = (vocab + len - 1) / len;
  return Geometry{static_cast<int>(nc), len};
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

size_t workspace_bytes(int64_t rows, int64_t vocab, int k) {
  const Geometry g = frontier_geometry(rows, vocab);
  return align256(size_t(rows + 1) * 4) + align256(size_t(rows) * g.num_chunks * sizeof(float2)) +
         align256(size_t(rows) * g.num_chunks * k * sizeof(uint64_t));
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" int64_t atlas_frontier_workspace_bytes(int64_t rows, int64_t vocab, int k) {
  if (rows <= 0 || vocab <= 0 || k <= 0 || k > kMaxK) return ATLAS_EINVAL;
  return static_cast<int64_t>(workspace_bytes(rows, vocab, std::min<int64_t>(k, vocab)));
}

static int check_cols(const CandCols& c) {
  ATLAS_REQUIRE(c.parent && c.root && c.token && c.rank && c.cum && c.plp, "candidate columns must not be NULL");
  return ATLAS_OK;
}

extern "C" int atlas_frontier_topk(const void* logits, int64_t rows, int64_t vocab, int64_t row_stride, int dtype,
                                   const float* proposal, int64_t proposal_stride, int k,
                                   const int64_t* parent_info_dev, int select_mode, int64_t num_selected,
                                   const int64_t* node_ids_dev, int64_t num_node_ids, void* token_logprobs_out,
                                   int64_t* token_ids_out, int64_t* records_out, int64_t* parent_rows_out,
                                   int64_t* selected_out, void* workspace_dev, size_t workspace_bytes_given,
                                   void* stream) {
  ATLAS_REQUIRE(logits && token_logprobs_out && token_ids_out && workspace_dev,
                "logits, outputs and workspace must not be NULL");
  ATLAS_REQUIRE(rows > 0 && rows <= 65535, "rows must be in 1..65535, got %lld", (long long)rows);
  ATLAS_REQUIRE(vocab > 0 && vocab < (int64_t(1) << 31), "vocab out of range");
  ATLAS_REQUIRE(k > 0 && k <= kMaxK && k <= vocab, "k must be in 1..min(%d, vocab), got %d", kMaxK, k);
  ATLAS_REQUIRE(dtype == ATLAS_DTYPE_F16 || dtype == ATLAS_DTYPE_BF16 || dtype == ATLAS_DTYPE_F32, "bad dtype");
  ATLAS_REQUIRE(row_stride >= vocab, "row_stride must be >= vocab");
  ATLAS_REQUIRE(proposal == nullptr || proposal_stride >= vocab, "proposal_stride must be >= vocab");
  ATLAS_REQUIRE(select_mode == ATLAS_FRONTIER_NONE || select_mode == ATLAS_FRONTIER_SELECT_GLOBAL ||
                    select_mode == ATLAS_FRONTIER_SELECT_PER_ROOT || select_mode == ATLAS_FRONTIER_PACK,
                "bad select_mode %d", select_mode);
  const int64_t count = rows * k;
  const bool want_records = records_out != nullptr;
  ATLAS_REQUIRE(!want_records || parent_info_dev != nullptr, "records need parent_info");
  ATLAS_REQUIRE(select_mode == ATLAS_FRONTIER_NONE || want_records, "selection writes records");
  ATLAS_REQUIRE(select_mode != ATLAS_FRONTIER_SELECT_GLOBAL && select_mode != ATLAS_FRONTIER_SELECT_PER_ROOT ||
                    (selected_out != nullptr && num_selected > 0),
                "selection needs selected_out and num_selected > 0");
  ATLAS_REQUIRE(select_mode != ATLAS_FRONTIER_PACK, "the fused launch selects; pack a given selection with "
                                                    "atlas_candidate_select");
  ATLAS_REQUIRE(!want_records || count <= kMaxCand, "at most %d candidates, got %lld", kMaxCand, (long long)count);
  ATLAS_REQUIRE(num_node_ids >= 0 && (num_node_ids == 0 || node_ids_dev != nullptr), "bad node ids");
  ATLAS_REQUIRE(num_node_ids == 0 || want_records, "node ids go into the records");
  ATLAS_REQUIRE((reinterpret_cast<uintptr_t>(workspace_dev) & 255) == 0, "workspace must be 256-byte aligned");
  ATLAS_REQUIRE(workspace_bytes_given >= workspace_bytes(rows, vocab, k), "workspace too small (%zu < %zu)",
                workspace_bytes_given, workspace_bytes(rows, vocab, k));

  const int esize = dtype == ATLAS_DTYPE_F32 ? 4 : 2;
  const Geometry g = frontier_geometry(rows, vocab);
  char* ws = static_cast<char*>(workspace_dev);
  FrontierArgs a{};
  a.logits = static_cast<const char*>(logits);
  a.row_stride_bytes = row_stride * esize;
  a.vocab = vocab;
  a.proposal = proposal;
  a.proposal_stride = proposal_stride;
  a.rows = static_cast<int>(rows);
  a.k = k;
  a.num_chunks = g.num_chunks;
  a.chunk_len = g.chunk_len;
  a.parent_info = parent_info_dev;
  a.token_logprobs = token_logprobs_out;
  a.token_ids = token_ids_out;
  a.parent_rows = parent_rows_out;
  a.counters = reinterpret_cast<int32_t*>(ws);
  ws += align256(size_t(rows + 1) * 4);
  a.stats = reinterpret_cast<float2*>(ws);
  ws += align256(size_t(rows) * g.num_chunks * sizeof(float2));
  a.lists = reinterpret_cast<uint64_t*>(ws);
  SelectArgs& s = a.sel;
  s.mode = want_records ? select_mode : -1;
  if (want_records) {
    // the candidates' columns are the records' columns 1..6
    s.cols.parent = records_out + 1;
    s.cols.root = records_out + 2;
    s.cols.token = records_out + 3;
    s.cols.rank = records_out + 4;
    s.cols.cum = reinterpret_cast<const double*>(records_out + 5);
    s.cols.plp = reinterpret_cast<const double*>(records_out + 6);
    s.cols.s_parent = s.cols.s_root = s.cols.s_token = s.cols.s_rank = s.cols.s_cum = s.cols.s_plp = 8;
    s.count = count;
    s.num_selected = num_selected;
    s.node_ids = node_ids_dev;
    s.num_node_ids = num_node_ids;
    s.selected_out = selected_out;
    s.records = records_out;
    s.records_filled = true;
    if (select_mode == ATLAS_FRONTIER_NONE) s.mode = ATLAS_FRONTIER_PACK;  // order column all -1
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DTYPE_F16) return launch_frontier<ATLAS_DTYPE_F16>(a, st);
  if (dtype == ATLAS_DTYPE_BF16) return launch_frontier<ATLAS_DTYPE_BF16>(a, st);
  return launch_frontier<ATLAS_DTYPE_F32>(a, st);
}

extern "C" int atlas_candidate_select(const int64_t* parent_route_ids, const int64_t* stage1_root_ids,
                                      const int64_t* pending_token_ids, const int64_t* ranks_in_parent,
                                      const double* cumulative_logprobs, const double* parent_logprobs,
                                      const int64_t* strides, int64_t count, int mode, int64_t num_selected,
                                      const int64_t* selected_in_dev, int64_t num_selected_in,
                                      const int64_t* node_ids_dev, int64_t num_node_ids, int64_t* order_out,
                                      int64_t* selected_out, int64_t* records_out, void* stream) {
  ATLAS_REQUIRE(strides != nullptr, "strides must not be NULL");
  ATLAS_REQUIRE(count >= 0 && count <= kMaxCand, "at most %d candidates, got %lld", kMaxCand, (long long)count);
  ATLAS_REQUIRE(mode >= ATLAS_FRONTIER_ORDER && mode <= ATLAS_FRONTIER_PACK, "bad mode %d", mode);
  ATLAS_REQUIRE(num_node_ids >= 0 && (num_node_ids == 0 || node_ids_dev != nullptr), "bad node ids");
  SelectArgs a{};
  a.cols = CandCols{parent_route_ids, stage1_root_ids, pending_token_ids, ranks_in_parent, cumulative_logprobs,
                    parent_logprobs, strides[0], strides[1], strides[2], strides[3], strides[4], strides[5]};
  if (count > 0) {
    const int rc = check_cols(a.cols);
    if (rc != ATLAS_OK) return rc;
  }
  a.count = count;
  a.mode = mode;
  a.num_selected = num_selected;
  a.selected_in = selected_in_dev;
  a.num_selected_in = num_selected_in;
  a.node_ids = node_ids_dev;
  a.num_node_ids = num_node_ids;
  a.order_out = order_out;
  a.selected_out = selected_out;
  a.records = records_out;
  a.records_filled = false;
  if (mode == ATLAS_FRONTIER_ORDER || mode == ATLAS_FRONTIER_ORDER_BY_ROOT)
    ATLAS_REQUIRE(order_out != nullptr, "order modes need order_out");
  if (mode == ATLAS_FRONTIER_SELECT_GLOBAL || mode == ATLAS_FRONTIER_SELECT_PER_ROOT)
    ATLAS_REQUIRE(selected_out != nullptr && num_selected > 0, "selection needs selected_out and num_selected > 0");
  if (mode == ATLAS_FRONTIER_PACK)
    ATLAS_REQUIRE(records_out != nullptr && (num_selected_in == 0 || selected_in_dev != nullptr),
                  "pack needs records_out and the selection");
  if (count == 0 && num_node_ids == 0) return ATLAS_OK;
  hipLaunchKernelGGL(candidate_select_kernel, dim3(1), dim3(kFThreads), 0, static_cast<hipStream_t>(stream), a);
  return launch_status("candidate_select_kernel");
}
