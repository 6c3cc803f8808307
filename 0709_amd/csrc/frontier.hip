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
//                          for another; the hand-offs are agent-scope atomic
//                          stores and loads, see publish_i64).
// The ordering works on any candidate batch as its own launch too
// (candidate_select_kernel).
#include "common.hpp"

namespace atlas {
namespace {

constexpr int kFThreads = 256;
constexpr int kMaxK = ATLAS_MAX_FRONTIER_K;
constexpr int kMaxCand = ATLAS_MAX_FRONTIER_CANDIDATES;
constexpr int kMaxChunks = kFThreads;  // the row merge gives each chunk list one thread
constexpr int kTile = 256;             // candidates per LDS tile of the ordering
constexpr int kFewMax = 64;            // global selections of up to this many take the bounded path
constexpr float kLog2e = 1.4426950408889634f;

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
    decode(__builtin_bit_cast(__attribute__((ext_vector_type(4))) uint32_t, u));
  }
  __device__ __forceinline__ void decode(__attribute__((ext_vector_type(4))) uint32_t u) {
    const uint32_t w[4] = {u[0], u[1], u[2], u[3]};
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

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
constexpr int kRegGroups = 8;  // 16-byte groups per thread a register-held chunk has at most

// A chunk of a 16-byte aligned row held in registers: thread t holds groups
// t, t + kFThreads, ... (all loads issued together, so a caller can start
// them before it waits for anything else); chunks of at most
// kRegGroups * kFThreads groups.
template <int DT>
struct ChunkRegs {
  static constexpr int E = Group<DT>::kElems;
  static constexpr int ES = DT == ATLAS_DTYPE_F32 ? 4 : 2;
  u32x4v v[kRegGroups];
  int64_t c0, c1, ng;
  __device__ __forceinline__ void load(const char* row, int64_t c0_, int64_t c1_) {
    c0 = c0_;
    c1 = c1_;
    ng = (c1 - c0) / E;
    if (ng == 0) return;
#pragma unroll
    for (int i = 0; i < kRegGroups; ++i) {
      // clamped, unconditional: every load of the batch is issued back to back
      const int64_t g = min<int64_t>(threadIdx.x + int64_t(i) * kFThreads, ng - 1);
      v[i] = *reinterpret_cast<const u32x4v*>(row + (c0 + g * E) * ES);
    }
  }
  // f(index, value) over the chunk; the tail past the last whole group is read
  // element by element.
  template <typename F>
  __device__ __forceinline__ void visit(const char* row, F&& f) const {
#pragma unroll
    for (int i = 0; i < kRegGroups; ++i) {
      const int64_t g = threadIdx.x + int64_t(i) * kFThreads;
      if (g < ng) {
        Group<DT> x;
        x.decode(v[i]);
#pragma unroll
        for (int e = 0; e < E; ++e) f(c0 + g * E + e, x.x[e]);
      }
    }
    for (int64_t i = c0 + ng * E + threadIdx.x; i < c1; i += kFThreads) f(i, load_one<DT>(row, i));
  }
};

// ---------------------------------------------------------------- reductions
// Wave reductions through DPP lane moves (no LDS round trips): swap within
// pairs and quads, mirror within 8 and 16 lanes, then row 0 into row 1 and
// row 2 into row 3 (row_bcast15), rows 0-1 into rows 2-3 (row_bcast31); lane
// 63 ends with the whole wave, which readlane hands to every lane.  Lanes a
// broadcast step leaves out receive `identity`.
constexpr int kDppXor1 = 0xB1;     // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;     // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppBcast15 = 0x142;
constexpr int kDppBcast31 = 0x143;

template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp32(uint32_t identity, uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(identity), static_cast<int>(v), CTRL, ROWS, 0xf, false));
}

template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t dpp64(uint64_t identity, uint64_t v) {
  const uint32_t lo = dpp32<CTRL, ROWS>(uint32_t(identity), uint32_t(v));
  const uint32_t hi = dpp32<CTRL, ROWS>(uint32_t(identity >> 32), uint32_t(v >> 32));
  return (uint64_t(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = umax64(v, dpp64<kDppXor1, 0xf>(0, v));
  v = umax64(v, dpp64<kDppXor2, 0xf>(0, v));
  v = umax64(v, dpp64<kDppHalfMirror, 0xf>(0, v));
  v = umax64(v, dpp64<kDppMirror, 0xf>(0, v));
  v = umax64(v, dpp64<kDppBcast15, 0xa>(0, v));
  v = umax64(v, dpp64<kDppBcast31, 0xc>(0, v));
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(uint32_t(v)), 63);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(uint32_t(v >> 32)), 63);
  return (uint64_t(hi) << 32) | lo;
}

// Hand-off between workgroups of one launch without an L2 write-back: the
// values another workgroup reads are stored and loaded as agent-scope atomics
// (coherent across the XCDs' L2s), and a writer waits until its stores are
// acknowledged before it counts itself in with a relaxed agent-scope add.  (An
// agent-scope release fence would write back the XCD's whole L2 in every
// workgroup.)
__device__ __forceinline__ void publish_i64(int64_t* p, int64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int64_t fetch_i64(const int64_t* p) {
  return __hip_atomic_load(const_cast<int64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() {
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0)
}
// Counts the calling workgroup in (after every thread's wait_stores and a
// barrier); true in the workgroup that arrives last of `total`.
__device__ __forceinline__ bool arrive_last(int32_t* counter, int total, int* flag) {
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
  __syncthreads();
  return *flag != 0;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
  v += static_cast<int>(dpp32<kDppXor1, 0xf>(0u, static_cast<uint32_t>(v)));
  v += static_cast<int>(dpp32<kDppXor2, 0xf>(0u, static_cast<uint32_t>(v)));
  v += static_cast<int>(dpp32<kDppHalfMirror, 0xf>(0u, static_cast<uint32_t>(v)));
  v += static_cast<int>(dpp32<kDppMirror, 0xf>(0u, static_cast<uint32_t>(v)));
  v += static_cast<int>(dpp32<kDppBcast15, 0xa>(0u, static_cast<uint32_t>(v)));
  v += static_cast<int>(dpp32<kDppBcast31, 0xc>(0u, static_cast<uint32_t>(v)));
  return __builtin_amdgcn_readlane(v, 63);
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
    s = s * __builtin_amdgcn_exp2f((m - m2) * kLog2e) + s2;
    m = m2;
  } else {
    s = s + s2 * __builtin_amdgcn_exp2f((m2 - m) * kLog2e);
  }
}

template <int CTRL, int ROWS>
__device__ __forceinline__ void ms_dpp(float& m, float& s) {
  const float m2 = __uint_as_float(dpp32<CTRL, ROWS>(__float_as_uint(-INFINITY), __float_as_uint(m)));
  const float s2 = __uint_as_float(dpp32<CTRL, ROWS>(0u, __float_as_uint(s)));
  ms_add(m, s, m2, s2);
}

// Block combine of per-thread (m, s) in a fixed order (the wave's DPP steps,
// then waves 0..3), so every workgroup of a row derives the same result.
__device__ __forceinline__ void block_ms(float& m, float& s, float* red) {
  ms_dpp<kDppXor1, 0xf>(m, s);
  ms_dpp<kDppXor2, 0xf>(m, s);
  ms_dpp<kDppHalfMirror, 0xf>(m, s);
  ms_dpp<kDppMirror, 0xf>(m, s);
  ms_dpp<kDppBcast15, 0xa>(m, s);
  ms_dpp<kDppBcast31, 0xc>(m, s);
  m = __uint_as_float(__builtin_amdgcn_readlane(static_cast<int>(__float_as_uint(m)), 63));
  s = __uint_as_float(__builtin_amdgcn_readlane(static_cast<int>(__float_as_uint(s)), 63));
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
  bool coherent;  // written by other workgroups of this launch: agent-scope loads
};

__device__ __forceinline__ int64_t col_i64(const int64_t* p, bool coherent) {
  return coherent ? fetch_i64(p) : *p;
}
__device__ __forceinline__ double col_f64(const double* p, bool coherent) {
  return coherent ? __longlong_as_double(fetch_i64(reinterpret_cast<const int64_t*>(p))) : *p;
}

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
  r.root = col_i64(c.root + i * c.s_root, c.coherent);
  r.cum = dorder(col_f64(c.cum + i * c.s_cum, c.coherent));
  r.parent = col_i64(c.parent + i * c.s_parent, c.coherent);
  r.rank = col_i64(c.rank + i * c.s_rank, c.coherent);
  r.token = col_i64(c.token + i * c.s_token, c.coherent);
  return r;
}

// LDS of the ordering: a tile of candidates by column (the score first, the
// other keys read only on equal scores), and per candidate its position and
// selection order (16 bits: at most 4096 candidates).
struct SelectSmem {
  uint64_t cum[kTile];
  int64_t root[kTile];
  int64_t parent[kTile];
  int64_t rank[kTile];
  int64_t token[kTile];
  int16_t pos[kMaxCand];  // position in the order (per root: inside the candidate's root)
  int16_t sel[kMaxCand];  // selection order, or -1
  // global top-n with small n: wave lists of the threads' best scores, the
  // bound, and the candidates at or above it with their counts
  uint64_t wave_best[kFThreads / 64][kFewMax];
  uint64_t bound;
  int num_few;
  int few[kFewMax * 4];
  int few_count[kFewMax * 4];
};
static_assert(kMaxCand <= 32767, "positions are 16-bit");

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

__device__ __forceinline__ void load_tile(const SelectArgs& a, SelectSmem& sm, int64_t t0, int n) {
  for (int j = threadIdx.x; j < n; j += kFThreads) {
    const Cand x = load_cand(a.cols, t0 + j);
    sm.cum[j] = x.cum;
    sm.root[j] = x.root;
    sm.parent[j] = x.parent;
    sm.rank[j] = x.rank;
    sm.token[j] = x.token;
  }
}

// Position of every candidate in the order: the number of candidates that
// come before it.  Keys: stage-1 root ascending (by_root), cumulative log-prob
// descending, parent route, rank in parent, token id ascending, then the
// original index (a stable sort's order).  within_root: count only the
// candidates of the same root.  One workgroup of kFThreads.
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
      load_tile(a, sm, t0, n);
      __syncthreads();
      if (!mine) continue;
      // Branch-free and unrolled, so the LDS reads of several candidates are
      // in flight together (equal scores are common: 16-bit log-probs).
#pragma unroll 8
      for (int j = 0; j < n; ++j) {
        const int64_t rj = sm.root[j];
        const uint64_t cj = sm.cum[j];
        const int64_t pj = sm.parent[j], kj = sm.rank[j], tj = sm.token[j];
        const bool same = !by_root || rj == me.root;
        const bool tie_first = pj < me.parent ||
                               (pj == me.parent && (kj < me.rank || (kj == me.rank && (tj < me.token ||
                                                                                       (tj == me.token && t0 + j < c)))));
        const bool b = same ? (cj > me.cum || (cj == me.cum && tie_first)) : (!within_root && rj < me.root);
        before += b ? 1 : 0;
      }
    }
    if (mine) sm.pos[c] = static_cast<int16_t>(before);
  }
  __syncthreads();
}

// Global top-n for n <= kFewMax.  T = the n-th largest of the threads' best
// scores is at most the n-th best score (n candidates reach it), so only
// candidates scoring at least T can be among the first n.  Those (few; at
// most 4 * kFewMax, else false) get their exact positions, each counted by
// the 64 lanes of one wave over all candidates.
__device__ bool select_global_few(const SelectArgs& a, SelectSmem& sm) {
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int64_t C = a.count;
  const int n = static_cast<int>(a.num_selected);
  uint64_t head = 0;
  for (int64_t c = t; c < C; c += kFThreads)
    head = umax64(head, dorder(col_f64(a.cols.cum + c * a.cols.s_cum, a.cols.coherent)));
  if (t == 0) sm.num_few = 0;
  for (int r = 0; r < n; ++r) {
    const uint64_t m = wave_max_u64(head);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(head == m && m != 0);
    if (hit != 0 && lane == __builtin_ctzll(hit)) head = 0;
    if (lane == 0) sm.wave_best[wave][r] = m;
  }
  __syncthreads();
  if (wave == 0) {
    int p = 0;
    head = lane < kFThreads / 64 ? sm.wave_best[lane][0] : 0;
    for (int r = 0; r < n; ++r) {
      const uint64_t m = wave_max_u64(head);
      const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < kFThreads / 64 && head == m && m != 0);
      if (hit != 0 && lane == __builtin_ctzll(hit)) {
        ++p;
        head = p < n ? sm.wave_best[lane][p] : 0;
      }
      if (lane == 0 && r == n - 1) sm.bound = m;
    }
  }
  __syncthreads();
  const uint64_t bound = sm.bound;
  for (int64_t c = t; c < C; c += kFThreads) {
    sm.sel[c] = -1;
    if (dorder(col_f64(a.cols.cum + c * a.cols.s_cum, a.cols.coherent)) >= bound) {
      const int i = atomicAdd(&sm.num_few, 1);
      if (i < kFewMax * 4) {
        sm.few[i] = static_cast<int>(c);
        sm.few_count[i] = 0;
      }
    }
  }
  __syncthreads();
  const int nf = sm.num_few;
  if (nf > kFewMax * 4) return false;
  for (int64_t t0 = 0; t0 < C; t0 += kTile) {
    const int nt = static_cast<int>(min<int64_t>(kTile, C - t0));
    __syncthreads();
    load_tile(a, sm, t0, nt);
    __syncthreads();
    for (int f = wave; f < nf; f += kFThreads / 64) {
      const int64_t c = sm.few[f];
      const Cand me = load_cand(a.cols, c);
      int before = 0;
      for (int j = lane; j < nt; j += 64) {
        const uint64_t cj = sm.cum[j];
        const int64_t pj = sm.parent[j], kj = sm.rank[j], tj = sm.token[j];
        const bool tie_first = pj < me.parent ||
                               (pj == me.parent && (kj < me.rank || (kj == me.rank && (tj < me.token ||
                                                                                       (tj == me.token && t0 + j < c)))));
        before += (cj > me.cum || (cj == me.cum && tie_first)) ? 1 : 0;
      }
      before = wave_sum_i32(before);
      if (lane == 0) sm.few_count[f] += before;
    }
  }
  __syncthreads();
  for (int f = t; f < nf; f += kFThreads) {
    const int p = sm.few_count[f];
    if (p < n) {
      const int c = sm.few[f];
      sm.sel[c] = static_cast<int16_t>(p);
      a.selected_out[p] = c;
    }
  }
  return true;
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
      if (a.num_selected <= kFewMax && select_global_few(a, sm)) break;
      count_before(a, sm, false, false);
      for (int64_t c = t; c < C; c += kFThreads) {
        const int p = sm.pos[c];
        const bool chosen = p < a.num_selected;
        sm.sel[c] = static_cast<int16_t>(chosen ? p : -1);
        if (chosen) a.selected_out[p] = c;
      }
      break;
    case kSelectPerRoot:
      count_before(a, sm, true, true);
      // selection offset of a root = the selected candidates of lower roots
      for (int64_t base = 0; base < C; base += kFThreads) {
        const int64_t c = base + t;
        const bool mine = c < C;
        const int64_t my_root = mine ? col_i64(a.cols.root + c * a.cols.s_root, a.cols.coherent) : 0;
        int off = 0;
        for (int64_t t0 = 0; t0 < C; t0 += kTile) {
          const int n = static_cast<int>(min<int64_t>(kTile, C - t0));
          __syncthreads();
          for (int j = t; j < n; j += kFThreads) sm.root[j] = col_i64(a.cols.root + (t0 + j) * a.cols.s_root, a.cols.coherent);
          __syncthreads();
          if (mine)
            for (int j = 0; j < n; ++j) off += (sm.root[j] < my_root && sm.pos[t0 + j] < a.num_selected) ? 1 : 0;
        }
        if (mine) {
          const int in_root = sm.pos[c];
          const bool chosen = in_root < a.num_selected;
          sm.sel[c] = static_cast<int16_t>(chosen ? off + in_root : -1);
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
          if (c >= 0 && c < C) sm.sel[c] = static_cast<int16_t>(i < 32767 ? i : -1);
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
  bool reg_chunks;  // chunks fit ChunkRegs (aligned rows use it)
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
  // Per thread: the maximum over its elements, then the sum of
  // exp2((x - max) * log2 e) over them -- from registers when the row is
  // aligned, else re-read from cache.
  float m = -INFINITY, s = 0.f;
  if (a.reg_chunks && (reinterpret_cast<uintptr_t>(rp) & 15) == 0) {
    ChunkRegs<DT> cr;
    cr.load(rp, c0, c1);
    cr.visit(rp, [&](int64_t, float x) { m = fmaxf(m, x); });
    if (m != -INFINITY) {
      const float mb = m * kLog2e;
      cr.visit(rp, [&](int64_t, float x) { s += __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -mb)); });
    }
  } else {
    for_chunk<DT>(rp, c0, c1, [&](int64_t, float x) { m = fmaxf(m, x); });
    if (m != -INFINITY) {
      const float mb = m * kLog2e;
      for_chunk<DT>(rp, c0, c1,
                    [&](int64_t, float x) { s += __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -mb)); });
    }
  }
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
  const int64_t c0 = int64_t(chunk) * a.chunk_len;
  const int64_t c1 = min(a.vocab, c0 + a.chunk_len);
  // The chunk's loads go out before the wait for the row statistics.
  const bool regs = a.reg_chunks && a.proposal == nullptr && (reinterpret_cast<uintptr_t>(rp) & 15) == 0;
  ChunkRegs<DT> cr;
  if (regs) cr.load(rp, c0, c1);

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

  TopList<KM> L;
  L.clear();
  // log_softmax rounded to the logits dtype: ((x - max) - lse)
  auto push_lp = [&](int64_t i, float x) { L.push(token_key(round_dt<DT>((x - row_max) - lse), uint32_t(i)), k); };
  if (regs) {
    // Each thread's largest logit (the first of equal ones) is an element of
    // the chunk, so the k-th largest of their keys bounds the chunk's k-th
    // key from below.  Only elements whose unrounded log-prob can round up to
    // the bound's value compute a key (a margin over half a 16-bit ulp), so
    // the insertion work no longer runs for almost every element.
    float mx = -INFINITY;
    int64_t mi = -1;
    cr.visit(rp, [&](int64_t i, float x) {
      const bool up = x > mx;
      mx = up ? x : mx;
      mi = up ? i : mi;
    });
    // (per wave: the k-th largest of its 64 keys bounds the chunk's k-th key
    // as well, without a barrier)
    uint64_t head = mi >= 0 ? token_key(round_dt<DT>((mx - row_max) - lse), uint32_t(mi)) : 0;
    uint64_t bound = 0;
    for (int r = 0; r < k; ++r) {
      bound = wave_max_u64(head);
      if (head == bound) head = 0;  // keys are distinct
    }
    float cut = -INFINITY;
    if (bound != 0) {
      const float lb = key_value(bound);
      cut = lb - (fabsf(lb) * 0x1p-6f + 1e-7f);
    }
    cr.visit(rp, [&](int64_t i, float x) {
      const float u = (x - row_max) - lse;
      if (u >= cut) L.push(token_key(round_dt<DT>(u), uint32_t(i)), k);
    });
  } else if (a.proposal == nullptr) {
    for_chunk<DT>(rp, c0, c1, push_lp);
  } else {
    const char* pp = reinterpret_cast<const char*>(a.proposal + int64_t(row) * a.proposal_stride);
    for_chunk<ATLAS_DTYPE_F32>(pp, c0, c1, [&](int64_t i, float x) { L.push(token_key(x, uint32_t(i)), k); });
  }
  block_topk<KM>(L, k, lists, wave_lists, best);
  int64_t* my_list = reinterpret_cast<int64_t*>(a.lists) + (int64_t(row) * a.num_chunks + chunk) * k;
  if (t < k) publish_i64(my_list + t, static_cast<int64_t>(best[t]));
  wait_stores();

  // Last chunk of the row merges the row.
  if (!arrive_last(&a.counters[row], a.num_chunks, &flag)) return;
  L.clear();
  if (t < a.num_chunks) {
    const int64_t* src = reinterpret_cast<const int64_t*>(a.lists) + (int64_t(row) * a.num_chunks + t) * k;
#pragma unroll
    for (int i = 0; i < KM; ++i)
      if (i < k) L.a[i] = static_cast<uint64_t>(fetch_i64(src + i));
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
      // columns the last row's workgroup reads go out as agent-scope stores
      int64_t* r = a.sel.records + c * 8;
      const int64_t* pi = a.parent_info + int64_t(row) * 3;
      const double plp = __longlong_as_double(pi[2]);
      r[0] = 0;
      publish_i64(r + 1, pi[0]);
      publish_i64(r + 2, pi[1]);
      publish_i64(r + 3, id);
      publish_i64(r + 4, t);
      publish_i64(r + 5, __double_as_longlong(plp + static_cast<double>(lp)));
      publish_i64(r + 6, pi[2]);
      // The order column belongs to the selecting workgroup whenever one
      // runs (it writes r[7] of every candidate, -1 included); a plain store
      // here as well would leave two XCDs' L2s holding the line dirty, and
      // the value that reaches memory would depend on their write-back order.
      if (a.sel.mode < 0) r[7] = -1;
    }
  }
  if (a.sel.mode < 0) return;
  wait_stores();

  // Last row orders and selects every candidate (best[] is read above before
  // the barrier that precedes the ordering's first use of the shared bytes).
  if (!arrive_last(&a.counters[a.rows], a.rows, &flag)) return;
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
  bool reg_chunks;
};

// Chunks of a multiple of 8 elements: about 512 (row, chunk) workgroups (all
// resident at once) but no more chunks than register-held chunks need
// (kRegGroups 16-byte groups per thread) unless the rows are few, at least
// ~512 elements, at most kMaxChunks per row.
Geometry frontier_geometry(int64_t rows, int64_t vocab, int esize) {
  constexpr int64_t kTargetGroups = 512;
  const int64_t reg_len = int64_t(kFThreads) * kRegGroups * (16 / esize);
  int64_t nc = (kTargetGroups + rows - 1) / rows;
  nc = std::min<int64_t>(nc, (vocab + 511) / 512);
  nc = std::max<int64_t>(nc, (vocab + reg_len - 1) / reg_len);
  nc = std::max<int64_t>(1, std::min<int64_t>(nc, kMaxChunks));
  int64_t len = (vocab + nc - 1) / nc;
  len = (len + 7) / 8 * 8;
  nc = (vocab + len - 1) / len;
  return Geometry{static_cast<int>(nc), len, len <= reg_len};
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

size_t workspace_bytes_for(int64_t rows, int64_t vocab, int k, int esize) {
  const Geometry g = frontier_geometry(rows, vocab, esize);
  return align256(size_t(rows + 1) * 4) + align256(size_t(rows) * g.num_chunks * sizeof(float2)) +
         align256(size_t(rows) * g.num_chunks * k * sizeof(uint64_t));
}

size_t workspace_bytes(int64_t rows, int64_t vocab, int k) {
  return std::max(workspace_bytes_for(rows, vocab, k, 2), workspace_bytes_for(rows, vocab, k, 4));
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
  const Geometry g = frontier_geometry(rows, vocab, esize);
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
  a.reg_chunks = g.reg_chunks;
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
    s.cols.coherent = true;
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
                    parent_logprobs, strides[0], strides[1], strides[2], strides[3], strides[4], strides[5], false};
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
