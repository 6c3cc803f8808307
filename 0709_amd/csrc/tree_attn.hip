// Ancestor-masked paged tree / forest verify attention for gfx950.
//
// A work item is a block of packed query rows (row = node * group +
// head_in_group, so the `group` query heads sharing a KV head are stacked as
// rows) of one KV head against one split of the request's keys; keys are
// processed in tiles of 64 gathered through the page table.  Two kernels:
//
//   tree_attn_d128_kernel  head_dim 128, pages of >= 16 tokens: 8 waves, KV
//                          streamed into a 4-tile LDS ring by direct
//                          global->LDS loads, V^T read with transposing LDS
//                          loads, scores of the next tile pipelined against
//                          the current tile's softmax (see its section below);
//   tree_attn_kernel       other shapes: 4 waves, KV staged through registers
//                          into LDS one tile ahead.
//
// MFMA formulation (v_mfma_f32_16x16x32 f16/bf16), per 16-row tile:
//   S^T[key, row] = K[key, :] . Q[row, :]     A = K from LDS, B = Q in registers
//   O^T[dim, row] += V^T[dim, key] . P^T[key, row]
// The C layout of a 16x16 MFMA gives lane l the column l % 16 and rows
// 4*(l/16)..+3, so every lane holds scores and outputs of a single query row:
// the online softmax needs only two cross-lane reductions (max) per tile and
// none for the rescale.  P^T feeds the second MFMA straight from registers
// because V^T is presented to it with its keys in the order in which the
// score tile's C layout hands them out (see vt_position).
//
// Masks are applied in registers: keys below mask_col_start are visible to
// every row, keys at and after it use the row's 64-bit ancestor bitmask; tiles
// wholly inside the always-visible range skip the mask code.
#include <mutex>

#include "common.hpp"

namespace atlas {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTileKeys = 64;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.0f;
// Largest row block of one work item: 16 row tiles of 16 (head_dim 128 with
// pages of >= 16 tokens); other shapes take up to 12 row tiles.
constexpr int kMaxRowsPerItem = 256;

struct AttnArgs {
  const char* q;
  int64_t q_stride_token;  // elements
  int64_t q_stride_head;   // elements
  const char* kv;
  int64_t page_stride;  // bytes
  int64_t v_offset;     // bytes
  int64_t token_stride; // bytes
  int64_t head_stride;  // bytes between a token's KV heads (head_dim * 2 for NHD pages, page_size * that for HND)
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* kv_len;
  const uint64_t* tree_mask;
  const int32_t* mask_col_start;
  const atlas_attn_work_t* work;
  const int32_t* page_window;  // per-item first page-id windows (64 ids), or null
  char* out;
  int64_t out_stride_token;  // elements
  int64_t out_stride_head;   // elements
  float* lse;
  uint16_t* part_o;  // normalised partial O rows in the output dtype
  float* part_lse;    // base-2 LSE of each partial row
  int64_t part_rows;  // rows the partial area holds; split rows at or past it are not written
  // Fused append (head_dim-128 kernel): K / V rows of each request's newest
  // qo_len tokens, [token, head, D] with these strides (elements), or null.
  const char* app_k;
  const char* app_v;
  int64_t app_stride_token;
  int64_t app_stride_head;
  // Rotary embedding of the fused step, or null: cos / sin rows [token, D]
  // (stride in elements, token index = the query row) rotate the queries as
  // they are read and the appended K rows before they are written.
  const char* rope_cos;
  const char* rope_sin;
  int64_t rope_stride_token;
  float scale_log2;  // sm_scale * log2(e)
  int mask_mode;
  // Tree mask words per query row: 1 = one ancestor word relative to the
  // request's mask_col_start; > 1 = one visibility word per 64-key tile from
  // the tile holding mask_col_start to the last key (wide trees, see
  // tile_mask_word).
  int mask_words;
  int group;
  int num_qo_heads;
  int page_size;
  int page_shift;
};

typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));

template <bool BF16>
struct Mfma;

// P is converted two values at a time; fp16 uses round-toward-zero packing
// (one instruction), bf16 round-to-nearest-even.  The row sum of the
// softmax is accumulated from the same packed values the P.V MFMA consumes.
template <>
struct Mfma<false> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  // K = 16 form: a and b hold four 16-bit elements each.
  static __device__ __forceinline__ f32x4 run16(v4i16 a, v4i16 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    _Float16 h = static_cast<_Float16>(x);
    return __builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
  }
  static __device__ __forceinline__ float sum2(uint32_t packed, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, packed), half2v{(_Float16)1.0f, (_Float16)1.0f}, acc,
                                  false);
  }
  // Fragments of a matrix of ones (the A operand that turns a P^T MFMA into
  // row sums).
  static __device__ __forceinline__ frag ones8() { return __builtin_bit_cast(frag, u16x8(0x3C00)); }
  static __device__ __forceinline__ v4i16 ones4() { return v4i16(short(0x3C00)); }
};

template <>
struct Mfma<true> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 run16(v4i16 a, v4i16 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    __bf16 h = static_cast<__bf16>(x);
    return __builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, bf16x2v{static_cast<__bf16>(a), static_cast<__bf16>(b)});
  }
  static __device__ __forceinline__ float sum2(uint32_t packed, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, packed),
                                           bf16x2v{(__bf16)1.0f, (__bf16)1.0f}, acc, false);
  }
  static __device__ __forceinline__ frag ones8() { return __builtin_bit_cast(frag, u16x8(0x3F80)); }
  static __device__ __forceinline__ v4i16 ones4() { return v4i16(short(0x3F80)); }
};

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// 16 bytes of KV, read once per launch: non-temporal, so they do not displace
// the queries, page ids and partial rows from the caches.
__device__ __forceinline__ uint4 load16_nt(const char* p) {
  const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
  return uint4{v[0], v[1], v[2], v[3]};
}

template <bool BF16>
__device__ __forceinline__ float half_to_float(uint32_t bits) {
  if constexpr (BF16) return __builtin_bit_cast(float, bits << 16);
  else return static_cast<float>(__builtin_bit_cast(_Float16, uint16_t(bits)));
}

// Rounds to the 16-bit type and back.
template <bool BF16>
__device__ __forceinline__ float round16(float x) {
  return half_to_float<BF16>(Mfma<BF16>::from_float(x));
}

// Rotary embedding of 8 consecutive 16-bit elements x at dims d .. d+7 with
// their rotate-half partners xp (dims d +- D/2) and the cos / sin of the same
// dims, rounded like the elementwise 16-bit tensor ops it replaces
// (q * cos + rotate_half(q) * sin, src/atlas_0709/flashinfer_full_verify.py:324-333):
// each product is rounded to the 16-bit type, then their sum.  rotate_half
// negates the second half, so the first half subtracts.  (A 16-bit product of
// 16-bit operands is exact in fp32 and fp32 carries more than 2p + 2 bits, so
// computing in fp32 and rounding once per op equals the 16-bit ops.)
template <bool BF16>
__device__ __forceinline__ u32x4v rope8(u32x4v x, u32x4v xp, u32x4v c, u32x4v s, bool first_half) {
  // Contracting a product into the sum (a 16-bit FMA) would skip its rounding.
#pragma clang fp contract(off)
  u32x4v r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t packed = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int sh = 16 * h;
      const float a = round16<BF16>(half_to_float<BF16>((x[i] >> sh) & 0xffffu) *
                                    half_to_float<BF16>((c[i] >> sh) & 0xffffu));
      const float b = round16<BF16>(half_to_float<BF16>((xp[i] >> sh) & 0xffffu) *
                                    half_to_float<BF16>((s[i] >> sh) & 0xffffu));
      packed |= uint32_t(Mfma<BF16>::from_float(first_half ? a - b : a + b)) << sh;
    }
    r[i] = packed;
  }
  return r;
}

// Visibility of the four keys p0 .. p0+3 a lane holds in one 16-key block
// (bit i for key p0 + i), branch-free: keys at or past kv_end are hidden; in
// tree mode keys below col0 (the prefix) are visible and key p >= col0 follows
// bit p - col0 of the row's ancestor word; in causal mode keys up to climit.
template <int MODE>
__device__ __forceinline__ uint32_t key_bits4(uint64_t tbits, int climit, int p0, int col0, int kv_end) {
  const int nlen = min(max(kv_end - p0, 0), 4);
  uint32_t vis = (1u << nlen) - 1u;
  if constexpr (MODE == ATLAS_MASK_TREE) {
    const int off = p0 - col0;
    const uint32_t up = off < 64 ? uint32_t(tbits >> (off & 63)) : 0u;  // off >= 0: bits off .. off+3
    const int k = min(max(-off, 0), 4);                                   // off < 0: k keys of the prefix
    const uint32_t down = uint32_t(tbits << (k & 63)) | ((1u << k) - 1u);
    vis &= (off >= 0 ? up : down) & 15u;
  } else if constexpr (MODE == ATLAS_MASK_CAUSAL) {
    const int nc = min(max(climit - p0 + 1, 0), 4);
    vis &= (1u << nc) - 1u;
  }
  return vis;
}
// Runtime mode without branches: every variant is computed and selected.
__device__ __forceinline__ uint32_t key_bits4(int mode, uint64_t tbits, int climit, int p0, int col0, int kv_end) {
  const uint32_t tree = key_bits4<ATLAS_MASK_TREE>(tbits, climit, p0, col0, kv_end);
  const uint32_t causal = key_bits4<ATLAS_MASK_CAUSAL>(tbits, climit, p0, col0, kv_end);
  const uint32_t none = key_bits4<ATLAS_MASK_NONE>(tbits, climit, p0, col0, kv_end);
  return mode == ATLAS_MASK_TREE ? tree : (mode == ATLAS_MASK_CAUSAL ? causal : none);
}

// Wide tree masks (more than 64 tree columns): the row's visibility word for
// the 64 keys of the tile starting at t0 (a multiple of 64): word
// t0 / 64 - col0 / 64 of the row's words, whose bit b covers key t0 + b
// (prefix keys set).  Tiles before the tree's first tile are wholly visible.
// Tested with key_bits4 against the window at t0 (col0 := t0).
__device__ __forceinline__ uint64_t tile_mask_word(const AttnArgs& a, int64_t row, int t0, int col0) {
  const int idx = (t0 >> 6) - (col0 >> 6);
  if (idx < 0) return ~0ull;
  if (idx >= a.mask_words) return 0ull;
  return a.tree_mask[row * a.mask_words + idx];
}

// Position inside a 32-key block of V^T at which key k (0..31) is stored.  The
// B operand of the P.V MFMA is built from two score tiles: lane group g holds
// keys 4g..4g+3 of the first tile and 16+4g..16+4g+3 of the second as its
// eight k-elements 8g..8g+7, so V^T stores key k at that same k-element.
__device__ __forceinline__ int vt_position(int k) {
  return ((k & 15) >> 2) * 8 + ((k >> 4) << 2) + (k & 3);
}

// Maxima of scores.  The IEEE maximum builtins map to v_maximum(3)_f32, which
// need no canonicalised operands (fmaxf makes the compiler quieten every MFMA
// result with an extra v_max_f32 first).  Scores are never NaN: masked keys
// are -inf, which every finite score exceeds.
__device__ __forceinline__ float max2f(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
// Maximum over the N scores of a lane: one three-input maximum per two values.
template <int N>
__device__ __forceinline__ float lane_max(const float (&v)[N]) {
  static_assert(N >= 2, "at least two values");
  float m = max2f(v[0], v[1]);
#pragma unroll
  for (int i = 2; i + 1 < N; i += 2) m = max3f(m, v[i], v[i + 1]);
  if constexpr (N % 2 == 1) m = max2f(m, v[N - 1]);
  return m;
}

// Reductions across the four 16-lane rows of a wave (lanes l, l^16, l^32,
// l^48) with the gfx950 row-swap permutes: swapping a register with itself
// yields each lane's value and its partner's, so no selection is needed.
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max2f(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max2f(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_max_across_groups(float v) { return xor32_max(xor16_max(v)); }
__device__ __forceinline__ float wave_sum_across_groups(float v) { return xor32_sum(xor16_sum(v)); }

// V^T row d stores its 16-byte granules XOR-swizzled by vt_swizzle(d): the
// eight rows one MFMA A-read touches per LDS cycle land in eight different
// granules, and the writers (rows 8c + e, c = 0..15) collide at most 2-way.
__device__ __forceinline__ int vt_swizzle(int d) { return (d ^ (d >> 3)) & 7; }

// Page-table walk of one thread's keys: key (t + key0) clamped to the split's
// last key, mapped to its physical page and in-page offset.
struct PageWalk {
  const int32_t* pages;
  int page_size;
  int page_shift;
  int last_key;
  int key0;

  __device__ __forceinline__ int clamp(int t) const { return min(t + key0, last_key); }
  __device__ __forceinline__ int page(int t) const {
    const int p = clamp(t);
    return pages[page_shift >= 0 ? (p >> page_shift) : (p / page_size)];
  }
  __device__ __forceinline__ const char* row(const char* base, int64_t page_stride, int64_t token_stride, int t,
                                             int phys_page) const {
    const int p = clamp(t);
    const int off = page_shift >= 0 ? (p & (page_size - 1)) : (p % page_size);
    return base + int64_t(phys_page) * page_stride + int64_t(off) * token_stride;
  }
};

// NWC waves compute, each owning RT row tiles of 16 rows (tile = wave +
// NWC * rt); all 4 waves load.  Rows beyond num_rows carry zero queries, so
// every MFMA runs unconditionally.
template <int D, bool BF16, int RT, int NWC>
__global__ __launch_bounds__(kThreads, (RT <= 2 ? 2 : 1)) void tree_attn_kernel(AttnArgs a) {
  typedef Mfma<BF16> M;
  typedef typename M::frag frag;
  constexpr int KS = D / 32;           // k-steps of the score MFMA
  constexpr int DT = D / 16;           // 16-dim output tiles
  constexpr int CH = D / 8;            // 16-byte chunks per key row
  constexpr int KROW = D + 8;          // K row stride in LDS (elements)
  constexpr int VROW = kTileKeys;      // V^T row stride in LDS (elements), swizzled granules
  constexpr int KPT = kTileKeys * CH / kThreads;  // consecutive keys per thread
  static_assert(KPT == 2 || KPT == 4, "head_dim must be 64 or 128");
  static_assert(NWC >= 1 && NWC <= kWaves, "compute waves");

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kTileKeys * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[D * VROW];

  const atlas_attn_work_t w = a.work[blockIdx.x];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = lane >> 4;
  const int r16 = lane & 15;

  const int kvh = w.kv_head;
  const int qo_start = w.qo_start;
  const int qo_len = w.qo_len;
  const int kv_len = w.kv_len;
  const int pt_base = w.page_offset;
  const int kv_end = min(w.kv_end, kv_len);
  const int G = a.group;
  const int64_t head_off = int64_t(kvh) * a.head_stride;

  // Keys < vis_all are visible to every row.
  int vis_all = kv_end;
  int col0 = 0;
  if (a.mask_mode == ATLAS_MASK_TREE) {
    col0 = w.mask_col_start;
    vis_all = min(vis_all, col0);
  } else if (a.mask_mode == ATLAS_MASK_CAUSAL) {
    vis_all = min(vis_all, kv_len - qo_len + 1);
  }

  const bool computes = wave < NWC;
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
    const int lr = (wave + NWC * rt) * 16 + r16;
    row_ok[rt] = computes && lr < w.num_rows;
    const int prow = w.row_start + (row_ok[rt] ? lr : 0);
    node_of[rt] = prow / G;
    head_of[rt] = kvh * G + (prow - node_of[rt] * G);
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const char* qrow = a.q + ((int64_t(qo_start + node_of[rt]) * a.q_stride_token +
                               int64_t(head_of[rt]) * a.q_stride_head) * 2);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 v = *reinterpret_cast<const uint4*>(qrow + (ks * 32 + grp * 8) * 2);
      if (!row_ok[rt]) v = uint4{0, 0, 0, 0};
      qf[rt][ks] = __builtin_bit_cast(frag, v);
    }
    tbits[rt] = (a.mask_mode == ATLAS_MASK_TREE && a.mask_words == 1 && row_ok[rt])
                    ? a.tree_mask[qo_start + node_of[rt]] : 0ull;
    climit[rt] = kv_len - qo_len + node_of[rt];
  }

  // Each thread stages KPT consecutive keys x one 16-byte chunk of K and V.
  const int chunk = tid % CH;
  const int key0 = (tid / CH) * KPT;
  const int last_key = kv_end - 1;
  const char* kv_head_base = a.kv + head_off + chunk * 16;

  const PageWalk pw{a.kv_indices + pt_base, a.page_size, a.page_shift, last_key, key0};
  // Empty splits (only for requests without keys) load nothing: the loop
  // below is skipped and the rows get O = 0, lse = -inf.
  const int t_first = w.kv_start < kv_end ? w.kv_start : kv_end;
  // A thread's KPT keys share one page whenever page_size is a multiple of
  // KPT (tiles start on multiples of 64): one page-table read per tile.
  const bool one_page = (a.page_size % KPT) == 0;
  int idx_cur = 0, idx_next = 0;
  uint4 kreg[KPT], vreg[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    kreg[j] = uint4{0, 0, 0, 0};
    vreg[j] = uint4{0, 0, 0, 0};
  }
  // Stage tile t: full tiles read KPT consecutive rows of one page; the
  // split's last partial tile clamps every key to the last valid key (rows of
  // valid memory and finite values; masked out of the softmax).
  auto stage = [](const PageWalk& pw, const char* base, int64_t page_stride, int64_t token_stride, int64_t v_off,
                  int t, int page0, bool full, bool one_page, uint4 (&kr)[KPT], uint4 (&vr)[KPT]) {
    if (full && one_page) {
      const int p = t + pw.key0;
      const int off = pw.page_shift >= 0 ? (p & (pw.page_size - 1)) : (p % pw.page_size);
      const char* r0 = base + int64_t(page0) * page_stride + int64_t(off) * token_stride;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        kr[j] = load16_nt(r0 + j * token_stride);
        vr[j] = load16_nt(r0 + j * token_stride + v_off);
      }
    } else {
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const char* rj = pw.row(base, page_stride, token_stride, t + j, pw.page(t + j));
        kr[j] = load16_nt(rj);
        vr[j] = load16_nt(rj + v_off);
      }
    }
  };
  if (t_first < kv_end) {
    idx_cur = pw.page(t_first);
    idx_next = pw.page(t_first + kTileKeys);
    stage(pw, kv_head_base, a.page_stride, a.token_stride, a.v_offset, t_first, idx_cur,
          t_first + kTileKeys <= kv_end, one_page, kreg, vreg);
  }

  const int vt_pos = (key0 >> 5) * 32 + vt_position(key0 & 31);

  for (int t0 = t_first; t0 < kv_end; t0 += kTileKeys) {
    __syncthreads();  // previous tile's LDS reads are done
#pragma unroll
    for (int j = 0; j < KPT; ++j)
      *reinterpret_cast<uint4*>(&k_lds[(key0 + j) * KROW + chunk * 8]) = kreg[j];
    {
      // Transpose KPT keys x 8 dims into 8 dim rows of KPT keys: byte
      // permutes pair the low (even dim) or high (odd dim) halves of two keys.
      constexpr uint32_t kLoLo = 0x05040100u, kHiHi = 0x07060302u;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const int word = d >> 1;
        const uint32_t sel = (d & 1) ? kHiHi : kLoLo;
        const int row = chunk * 8 + d;
        uint16_t* dst = &vt_lds[row * VROW + (((vt_pos >> 3) ^ vt_swizzle(row)) << 3) + (vt_pos & 7)];
        auto w4 = [&](int j) -> uint32_t {
          return word == 0 ? vreg[j].x : word == 1 ? vreg[j].y : word == 2 ? vreg[j].z : vreg[j].w;
        };
        if constexpr (KPT == 4) {
          *reinterpret_cast<uint2*>(dst) =
              uint2{__builtin_amdgcn_perm(w4(1), w4(0), sel), __builtin_amdgcn_perm(w4(3), w4(2), sel)};
        } else {
          *reinterpret_cast<uint32_t*>(dst) = __builtin_amdgcn_perm(w4(1), w4(0), sel);
        }
      }
    }
    __syncthreads();

    // Prefetch: the next tile's K/V with the page id fetched one tile
    // earlier, and the page id of the tile after it.
    {
      const int tn = t0 + kTileKeys;
      idx_cur = idx_next;
      idx_next = pw.page(tn + kTileKeys);
      if (tn < kv_end)
        stage(pw, kv_head_base, a.page_stride, a.token_stride, a.v_offset, tn, idx_cur, tn + kTileKeys <= kv_end,
              one_page, kreg, vreg);
    }

    if (!computes) continue;

    // ---- scores S^T = K Q^T ----
    f32x4 s[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[rt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      frag af[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        af[ks] = __builtin_bit_cast(
            frag, *reinterpret_cast<const uint4*>(&k_lds[(kt * 16 + r16) * KROW + ks * 32 + grp * 8]));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) s[rt][kt] = M::run(af[ks], qf[rt][ks], s[rt][kt]);
    }

    // ---- online softmax (lazy rescale), P^T fragments ----
    // Scores stay raw (unscaled) until exp2(fma(s, scale*log2e, -m)).
    const bool need_mask = (t0 + kTileKeys) > vis_all;
    frag pf[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if (need_mask) {
        uint64_t wbits = tbits[rt];
        int wcol0 = col0;
        if (a.mask_mode == ATLAS_MASK_TREE && a.mask_words > 1) {
          wbits = row_ok[rt] ? tile_mask_word(a, int64_t(qo_start + node_of[rt]), t0, col0) : 0ull;
          wcol0 = t0;
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const uint32_t vis = key_bits4(a.mask_mode, wbits, climit[rt], t0 + kt * 16 + grp * 4, wcol0, kv_end);
#pragma unroll
          for (int i = 0; i < 4; ++i) s[rt][kt][i] = ((vis >> i) & 1u) ? s[rt][kt][i] : -INFINITY;
        }
      }
      float sv[16];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[4 * kt + i] = s[rt][kt][i];
      const float mx = wave_max_across_groups(lane_max<16>(sv)) * a.scale_log2;
      // Lazy rescale: keep the running reference max until a row's max grows
      // by more than kRescaleLog2 (P stays below 2^kRescaleLog2), so most
      // tiles skip the O rescale.
      if (__builtin_amdgcn_ballot_w64(mx > m_run[rt] + kRescaleLog2) != 0) {
        const float m_new = fmaxf(m_run[rt], mx);
        const float alpha = (m_run[rt] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[rt] - m_new);
        l_run[rt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[rt][dt] *= alpha;
        m_run[rt] = m_new;
      }
      // A row with every key masked so far has m = -inf and only -inf scores.
      const float neg_m = m_run[rt] == -INFINITY ? 0.f : -m_run[rt];
      uint32_t pk[4][2];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][kt][0], a.scale_log2, neg_m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][kt][1], a.scale_log2, neg_m));
        const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][kt][2], a.scale_log2, neg_m));
        const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][kt][3], a.scale_log2, neg_m));
        pk[kt][0] = M::pack2(p0, p1);
        pk[kt][1] = M::pack2(p2, p3);
        l_run[rt] = M::sum2(pk[kt][1], M::sum2(pk[kt][0], l_run[rt]));
      }
      pf[rt][0] = __builtin_bit_cast(frag, uint4{pk[0][0], pk[0][1], pk[1][0], pk[1][1]});
      pf[rt][1] = __builtin_bit_cast(frag, uint4{pk[2][0], pk[2][1], pk[3][0], pk[3][1]});
    }

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      frag av[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        av[kk] = __builtin_bit_cast(
            frag, *reinterpret_cast<const uint4*>(
                      &vt_lds[(dt * 16 + r16) * VROW + (((kk * 4 + grp) ^ vt_swizzle(dt * 16 + r16)) << 3)]));
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) o[rt][dt] = M::run(av[kk], pf[rt][kk], o[rt][dt]);
    }
  }

  if (!computes) return;
  // ---- epilogue ----
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float l_tot = wave_sum_across_groups(l_run[rt]);
    if (!row_ok[rt]) continue;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const float lse2 = l_tot > 0.f ? m_run[rt] + __builtin_log2f(l_tot) : -INFINITY;
    const int lr = (wave + NWC * rt) * 16 + r16;
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
      if (prow >= a.part_rows) continue;
      char* po = reinterpret_cast<char*>(a.part_o + prow * D);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint32_t lo = uint32_t(M::from_float(o[rt][dt][0] * inv)) |
                            (uint32_t(M::from_float(o[rt][dt][1] * inv)) << 16);
        const uint32_t hi = uint32_t(M::from_float(o[rt][dt][2] * inv)) |
                            (uint32_t(M::from_float(o[rt][dt][3] * inv)) << 16);
        *reinterpret_cast<uint2*>(po + (dt * 16 + grp * 4) * 2) = uint2{lo, hi};
      }
      if (grp == 0) a.part_lse[prow] = lse2;
    }
  }
}

struct MergeArgs {
  const atlas_attn_merge_t* merge;
  const int32_t* qo_indptr;
  const uint16_t* part_o;
  const float* part_lse;
  int64_t part_rows;  // rows the partial area holds; items reaching past it are skipped
  char* out;
  int64_t out_stride_token;
  int64_t out_stride_head;
  float* lse;
  int group;
  int num_qo_heads;
};

// One wave per packed row, four rows per workgroup.  Lane (g, c) folds the
// 16-byte chunk c of splits g, g + G, g + 2G, ... (G = 64 / (D / 8) split
// groups) online, kMergeUnroll splits per round of independent loads (one
// round covers 32 splits at head_dim 128); the groups then combine through
// cross-lane reductions.  No LDS and no workgroup barriers, so a row costs
// the merge item load and one round of partial-state loads.
constexpr int kMergeThreads = 256;
constexpr int kMergeRowsPerBlock = kMergeThreads / 64;
constexpr int kMergeUnroll = 8;

// Eight 16-bit values (fp16 or bf16) to floats.
template <bool BF16>
__device__ __forceinline__ void unpack8(uint4 v, float (&f)[8]) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (BF16) {
      f[2 * i] = __uint_as_float(u[i] << 16);
      f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    } else {
      const half2v h = __builtin_bit_cast(half2v, u[i]);
      f[2 * i] = static_cast<float>(h[0]);
      f[2 * i + 1] = static_cast<float>(h[1]);
    }
  }
}

template <int CH>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (CH <= 8) v = fmaxf(v, __shfl_xor(v, 8));
  return wave_max_across_groups(v);
}
template <int CH>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (CH <= 8) v += __shfl_xor(v, 8);
  return wave_sum_across_groups(v);
}

// Merges the split states of packed row `row` of merge item `mi` and writes
// the final output row (and LSE), one wave per row.
template <int D, bool BF16>
__device__ __forceinline__ void merge_row(const MergeArgs& a, const atlas_attn_merge_t& mi, int row, int lane) {
  typedef Mfma<BF16> M;
  constexpr int CH = D / 8;   // 16-byte chunks per row
  constexpr int G = 64 / CH;  // split groups per wave
  static_assert(CH == 8 || CH == 16, "head_dim 64 or 128");
  const int g = lane / CH;
  const int c = lane % CH;
  const int ns = mi.num_splits;
  const int64_t base = int64_t(mi.partial_row) + row;

  float m_t = -INFINITY, wsum = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = g; s0 < ns; s0 += kMergeUnroll * G) {
    float l[kMergeUnroll];
    uint4 raw[kMergeUnroll];
#pragma unroll
    for (int k = 0; k < kMergeUnroll; ++k) {
      // Splits past the last re-read split s0 (always present) and are
      // given weight zero: unconditional loads stay in one batch, where a
      // guarded load would be followed by a wait of its own.
      const int sp = s0 + k * G;
      const int64_t r = base + int64_t(sp < ns ? sp : s0) * mi.num_rows;
      const float lv = a.part_lse[r];
      raw[k] = *reinterpret_cast<const uint4*>(a.part_o + r * D + c * 8);
      l[k] = sp < ns ? lv : -INFINITY;
    }
    float m_new = m_t;
#pragma unroll
    for (int k = 0; k < kMergeUnroll; ++k) m_new = max2f(m_new, l[k]);
    // No early exit on an all-masked round: a branch here would hold the O
    // loads back behind the LSE loads.  With m_new = -inf every weight is 0.
    const float sc = m_t == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_t - m_new);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= sc;
    wsum *= sc;
#pragma unroll
    for (int k = 0; k < kMergeUnroll; ++k) {
      const float wk = l[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(l[k] - m_new);
      float v[8];
      unpack8<BF16>(raw[k], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += wk * v[i];
      wsum += wk;
    }
    m_t = m_new;
  }
  const float mx = group_max<CH>(m_t);
  const float f = (m_t == -INFINITY || mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_t - mx);
  wsum = group_sum<CH>(wsum * f);
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = group_sum<CH>(acc[i] * f);
  if (g != 0) return;
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const int prow_q = mi.row_start + row;
  const int node = prow_q / a.group;
  const int head = mi.kv_head * a.group + (prow_q - node * a.group);
  const int qo_start = a.qo_indptr[mi.req];
  char* orow = a.out + ((int64_t(qo_start + node) * a.out_stride_token + int64_t(head) * a.out_stride_head) * 2);
  uint32_t pk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    pk[i] = uint32_t(M::from_float(acc[2 * i] * inv)) | (uint32_t(M::from_float(acc[2 * i + 1] * inv)) << 16);
  // 8-byte stores: output rows are only required to be 8-byte aligned.
  *reinterpret_cast<uint2*>(orow + c * 16) = uint2{pk[0], pk[1]};
  *reinterpret_cast<uint2*>(orow + c * 16 + 8) = uint2{pk[2], pk[3]};
  if (c == 0 && a.lse != nullptr)
    a.lse[int64_t(qo_start + node) * a.num_qo_heads + head] = wsum > 0.f ? (mx + __builtin_log2f(wsum)) * kLn2 : -INFINITY;
}

template <int D, bool BF16>
__global__ __launch_bounds__(kMergeThreads) void tree_attn_merge_kernel(MergeArgs a) {
  const atlas_attn_merge_t mi = a.merge[blockIdx.x];
  const int row = blockIdx.y * kMergeRowsPerBlock + (threadIdx.x >> 6);
  if (row >= mi.num_rows) return;
  if (mi.partial_row < 0 || int64_t(mi.partial_row) + int64_t(mi.num_splits) * mi.num_rows > a.part_rows) return;
  merge_row<D, BF16>(a, mi, row, threadIdx.x & 63);
}

// ---------------------------------------------------------------------------
// head_dim 128: KV streamed into LDS with direct global->LDS loads.
//
// The K and V rows of a 64-key tile land in LDS through
// global_load_lds_dwordx4 (each lane's 16 bytes go to the wave's 1 KiB block
// at its lane position), so no registers or VALU work stage the KV.  A ring
// of STAGES tiles keeps STAGES-1 tiles in flight while one is computed, with
// one barrier per tile.  Rows are row-major in LDS with their 16-byte granules
// XOR-swizzled by key: K by (key & 15), so the 16 keys a score-MFMA operand
// read touches hit 16 distinct granules; V by 2*(key & 7), so the transposing
// reads below spread over the banks.
//
// V^T for O^T += V^T P^T comes from ds_read_b64_tr_b16: within a 16-lane block,
// output lane i, element e is element (i % 4) of the 8 bytes that source lane
// 4e + i/4 addressed.  A lane with block index g and in-block index s = 4e + q
// addresses V[key][16*dt + 4q .. 4q + 3] with key = 32*kk + 4g + e (first read)
// or that key + 16 (second read), so output lane i holds V[key(g, e)][16dt + i]:
// the A operand of the MFMA with its eight k-elements in the key order of the
// score tile's C layout (keys 4g..4g+3 and 16+4g..16+4g+3 of the 32-key half).
// ---------------------------------------------------------------------------
constexpr int kRowBytes128 = 128 * 2;
constexpr int kHalf128 = kTileKeys * kRowBytes128;  // 16 KiB of K, then 16 KiB of V
constexpr int kTile128 = 2 * kHalf128;

__device__ __forceinline__ v4i16 lds_read_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)(reinterpret_cast<uintptr_t>(p)));
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt 7, lgkmcnt 15).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// 16 bytes from global memory into LDS at (wave-uniform base + 16 * lane).
// Issued as inline assembly so the compiler's wait-count pass, which would
// wait for every outstanding load before each LDS read, leaves the ring's
// in-flight tiles alone; the kernel waits for them explicitly (wait_vmcnt).
__device__ __forceinline__ void dma16(const char* gaddr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gaddr), "s"(lds_base) : "memory", "m0");
}

// KV rows are read once per launch, so their loads carry the non-temporal
// hint: they do not displace the queries, page ids and partial rows from the
// caches (1.2 us per layer less on the 16k forest).
__device__ __forceinline__ void dma16_kv(const char* gaddr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(gaddr), "s"(lds_base) : "memory", "m0");
}

// The KV load with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane
// offset: the base's arithmetic runs on the scalar unit, the offsets stay in
// registers for the whole loop.
__device__ __forceinline__ void dma16_s(const char* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}

// Issue the K and V rows of one tile into a stage: lane l of loader li loads,
// for each of its blocks b = NL*j + li, granule (l % 16) of the swizzled row of
// key 4b + l/16 into the 1 KiB block b of the K and V halves.
template <int NL>
__device__ __forceinline__ void issue_tile(const char* head_base, int64_t page_stride, int64_t token_stride,
                                           int64_t v_offset, const int (&pid)[16 / NL], int t0, int last_key,
                                           int page_size, int li, int lane, uint32_t stage) {
  const int c16p = lane & 15;
#pragma unroll
  for (int j = 0; j < 16 / NL; ++j) {
    const int blk = NL * j + li;
    const int key = 4 * blk + (lane >> 4);
    const int p = min(t0 + key, last_key);
    const char* row = head_base + int64_t(pid[j]) * page_stride + int64_t(p & (page_size - 1)) * token_stride;
    dma16_kv(row + ((c16p ^ (key & 15)) << 4), stage + blk * 1024);
    dma16_kv(row + v_offset + ((c16p ^ ((key & 7) << 1)) << 4), stage + kHalf128 + blk * 1024);
  }
}

// Per-item values every wave needs.
struct ItemCtx {
  int t_first, nt, nt_plain, kv_end, col0, qo_start, qo_len, kv_len;
  int win0;  // this lane's id of the item's first page-id window (plan-provided)
};

// What one workgroup streams: the split's tiles, their page ids and the LDS
// ring, plus this wave's loader index (li < 0: the wave issues no loads).
//
// Page ids reach a loader wave 64 at a time: lane l of `win_cur` holds the id
// of the split's page 64*win + l (clamped to its last page), `win_nxt` the
// next 64.  A tile's pages never straddle a window (a tile is 64 aligned keys,
// pages are a power of two >= 16 tokens), and the ids of a block are read with
// v_readlane, so the loop issues no scalar memory loads whose completion would
// be tied to the LDS reads' counter.
template <int NL>
struct Ring {
  const char* head_base;
  const int32_t* pages;  // the request's page ids
  int64_t page_stride, token_stride, v_offset;
  int page_size, page_shift;
  int t_first, nt, last_key;
  int nt_full;           // leading tiles whose 64 keys all lie before last_key + 1
  int page0, last_page;  // first and last page of the split
  int win;
  int win_cur, win_nxt;
  int li, lane;
  uint32_t lds0;
  // Lane offsets of the loader's blocks j inside their page (row within the
  // page plus the swizzled granule), K and V halves: the same on every tile
  // of a full tile (tiles start at multiples of 64 keys).
  uint32_t off_k[16 / NL], off_v[16 / NL];
};

template <int NL>
__device__ __forceinline__ int window_ids(const Ring<NL>& r, int w) {
  return r.pages[min(r.page0 + 64 * w + r.lane, r.last_page)];
}

// Vector loads of the first two page windows (loader waves); the caller waits
// for them together with the queries before the first tile is issued.
// win0: the item's first window when the plan provides it (loaded at
// workgroup start, before the work item arrived), else -1 (lane 0 decides).
// The second window is needed only by splits of more than 64 pages.
template <int NL>
__device__ __forceinline__ void ring_load_windows(Ring<NL>& r, bool have_win0, int win0) {
  r.win = 0;
  if (r.li >= 0 && r.nt > 0) {
    r.win_cur = have_win0 ? win0 : window_ids<NL>(r, 0);
    if (r.last_page - r.page0 >= 64) r.win_nxt = window_ids<NL>(r, 1);
  }
}

// The KV ring holds kStages128 tiles.  Tile k is issued at ring step k - 3;
// ring step t waits for tile t+1, joins the workgroup barrier and issues tile
// t+3 into the stage tile t-1 used.  Waves that pipeline the next tile's
// scores compute tile t after step t (reading tiles t and t+1); the others
// compute tile t before step t.  Either way every wave is past its last read
// of tile t-1 at step t's barrier.  (Issuing a third tile ahead, where no wave
// pipelines, measured slower: the extra loads in flight congest the paged
// stream.)
constexpr int kStages128 = 4;

template <int NL>
__device__ __forceinline__ void ring_issue(Ring<NL>& r, int k) {
  if (r.li >= 0 && k < r.nt) {
    const int t0 = r.t_first + k * kTileKeys;
    const int wk = ((t0 >> r.page_shift) - r.page0) >> 6;
    if (wk != r.win) {
      // Advance one window; the next one is needed no sooner than 16 tiles on.
      r.win = wk;
      r.win_cur = r.win_nxt;
      r.win_nxt = window_ids<NL>(r, wk + 1);
    }
    int pid[16 / NL];
#pragma unroll
    for (int j = 0; j < 16 / NL; ++j) {
      const int rel = (min(t0 + 4 * (NL * j + r.li), r.last_key) >> r.page_shift) - r.page0;
      pid[j] = __builtin_amdgcn_readlane(r.win_cur, rel & 63);
    }
    const uint32_t stage = r.lds0 + (k % kStages128) * kTile128;
    if (k < r.nt_full) {
      // A block's four keys share one page (pages hold >= 16 aligned keys),
      // so its row base is wave-uniform: page base + the tile's start inside
      // a page of more than 64 keys, on the scalar unit.
      const int64_t tile_in_page = int64_t(t0 & (r.page_size - 1) & ~(kTileKeys - 1)) * r.token_stride;
#pragma unroll
      for (int j = 0; j < 16 / NL; ++j) {
        const int blk = NL * j + r.li;
        const char* kbase = r.head_base + int64_t(pid[j]) * r.page_stride + tile_in_page;
        dma16_s(kbase, r.off_k[j], stage + blk * 1024);
        dma16_s(kbase + r.v_offset, r.off_v[j], stage + kHalf128 + blk * 1024);
      }
    } else {
      // The split's last, partial tile: keys past the last one re-read it.
      issue_tile<NL>(r.head_base, r.page_stride, r.token_stride, r.v_offset, pid, t0, r.last_key, r.page_size,
                     r.li, r.lane, stage);
    }
  }
}

__device__ __forceinline__ void bare_barrier() {
  // A bare s_barrier: the workgroup fence of __syncthreads would also wait
  // for the tiles still in flight.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Waits until tile `k` has landed given that tiles up to min(k + ahead, nt-1)
// were issued after it (ahead <= 2).  Waves that issue nothing have nothing
// outstanding, so the wait returns at once.
template <int NL>
__device__ __forceinline__ void ring_wait(int k, int ahead, int nt) {
  constexpr int L = 2 * (16 / NL);
  const int after = min(ahead, nt - 1 - k);
  if (after >= 2) wait_vmcnt<2 * L>();
  else if (after == 1) wait_vmcnt<L>();
  else wait_vmcnt<0>();
}

// Queries of the item's rows, staged through LDS at kQOffset (stage 3 and the
// 32 KiB past the ring): row r (local) is 256 bytes at kQOffset + 256 r with
// its 16-byte granules XOR-swizzled by (r & 15), rows past num_rows repeat the
// last row.  Loader li issues the 1 KiB blocks (four rows) li, li + NL, ...
constexpr int kQOffset = 3 * kTile128;
constexpr int kLdsBytes128 = kStages128 * kTile128 + 32 * 1024;

template <int NL>
__device__ __forceinline__ void issue_q(const Ring<NL>& r, const AttnArgs& a, const atlas_attn_work_t& w,
                                       const ItemCtx& c, int T) {
  const int gp = r.lane & 15;
  for (int i = r.li; i < 4 * T; i += NL) {
    const int row = 4 * i + (r.lane >> 4);
    const int pr = w.row_start + min(row, w.num_rows - 1);
    const int node = pr / a.group;
    const int head = w.kv_head * a.group + (pr - node * a.group);
    const char* src = a.q + ((int64_t(c.qo_start + node) * a.q_stride_token + int64_t(head) * a.q_stride_head) * 2);
    dma16(src + ((gp ^ (row & 15)) << 4), r.lds0 + kQOffset + i * 1024);
  }
}

// Loader waves: page windows first (waited alone), then tile 0, the queries
// and tiles 1, 2, so the KV stream starts one round trip after the work item
// and the queries land with tile 0.  (Issuing the queries ahead of the page
// window wait measured slower: they delay tile 0.)
template <int NL>
__device__ __forceinline__ void ring_begin(Ring<NL>& r, const AttnArgs& a, const atlas_attn_work_t& w,
                                           const ItemCtx& c, int T) {
  ring_load_windows<NL>(r, a.page_window != nullptr, c.win0);
  wait_vmcnt<0>();
  ring_issue<NL>(r, 0);
  if (r.li >= 0 && r.nt > 0) issue_q<NL>(r, a, w, c, T);
  ring_issue<NL>(r, 1);
  ring_issue<NL>(r, 2);
}

// Tile 0 landed (tiles 1 and 2 may be in flight).
template <int NL>
__device__ __forceinline__ void ring_first(const Ring<NL>& r) {
  ring_wait<NL>(0, 2, r.nt);
  bare_barrier();
}

template <int NL>
__device__ __forceinline__ void ring_step(Ring<NL>& r, int t) {
  if (t + 1 < r.nt) ring_wait<NL>(t + 1, 1, r.nt);
  bare_barrier();
  ring_issue<NL>(r, t + 3);
}

// A wave with no rows: loads its share of the tiles (if it is a loader) and
// keeps the workgroup's barrier count.
template <int NL>
__device__ __forceinline__ void ring_only(Ring<NL>& r, const AttnArgs& a, const atlas_attn_work_t& w,
                                          const ItemCtx& c, int T) {
  ring_begin<NL>(r, a, w, c, T);
  if (r.nt > 0) {
    ring_first<NL>(r);
    for (int t = 0; t < r.nt; ++t) ring_step<NL>(r, t);
  }
}

// Per-wave state of the row tiles a wave owns.
template <bool BF16, int RT>
struct RowState {
  typename Mfma<BF16>::frag qf[RT][4];
  f32x4 o[RT][8];
  float m_run[RT];
  // Row sums of P, accumulated by an MFMA of a ones matrix with P^T beside
  // the P.V MFMAs: every element holds the lane's row sum over all keys.
  f32x4 l_acc[RT];
  uint64_t tbits[RT];
  int climit[RT];
  int node_of[RT];
  int head_of[RT];
  int lrow[RT];  // row index inside the item
  bool row_ok[RT];
  // Rotary cos / sin of the lane's query granules (fused step with RoPE):
  // granule ks * 4 + grp of each row tile's node, live until d128_read_q.
  u32x4v rcos[RT][4];
  u32x4v rsin[RT][4];
};

// Scores S^T = K Q^T of the NKT 16-key blocks kb0 .. kb0+NKT-1 of one tile for
// a wave's RT row tiles (NKT = 4: the whole 64-key tile).
template <bool BF16, int RT, int NKT>
__device__ __forceinline__ void d128_scores(const RowState<BF16, RT>& st, const char* sb, int kb0, int grp, int r16,
                                            f32x4 (&s)[RT][NKT]) {
  typedef Mfma<BF16> M;
  typedef typename M::frag frag;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int j = 0; j < NKT; ++j) s[rt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < NKT; ++j) {
    const int kt = kb0 + j;
    frag af[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      af[ks] = __builtin_bit_cast(
          frag, *reinterpret_cast<const uint4*>(sb + (kt * 16 + r16) * kRowBytes128 + (((ks * 4 + grp) ^ r16) << 4)));
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) s[rt][j] = M::run(af[ks], st.qf[rt][ks], s[rt][j]);
  }
}

// Online softmax of the scores of blocks kb0 .. kb0+NKT-1 and O^T += V^T P^T
// with V^T from transposing LDS reads, in three phases so that a pipelining
// wave can place the next tile's score MFMAs between them:
//   d128_rowmax  mask (kMasked tiles), row maxima and the lazy rescale: the
//                running maximum moves only when a row's maximum grew by more
//                than kRescaleLog2 (P stays below 2^kRescaleLog2), so the
//                rescale of O and l, a branch, is skipped on most tiles;
//   d128_exp     P = exp2(s * scale - m), packed to 16 bits, row sums;
//   d128_pv      O^T += V^T P^T.
// d128_exp and d128_pv contain no branches: placed after d128_rowmax they
// form one basic block with whatever MFMAs the caller puts beside them.
constexpr int kPlain = 0;
constexpr int kMasked = 1;
template <bool BF16, int RT, int NKT, int MODE>
__device__ __forceinline__ void d128_rowmax(RowState<BF16, RT>& st, f32x4 (&s)[RT][NKT], int kb0, int t0,
                                            int kv_end, int col0, int mask_mode, float scale_log2, int grp) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if constexpr (MODE != kPlain) {
#pragma unroll
      for (int j = 0; j < NKT; ++j) {
        const uint32_t vis = key_bits4(mask_mode, st.tbits[rt], st.climit[rt], t0 + (kb0 + j) * 16 + grp * 4, col0,
                                       kv_end);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[rt][j][i] = ((vis >> i) & 1u) ? s[rt][j][i] : -INFINITY;
      }
    }
    float sv[4 * NKT];
#pragma unroll
    for (int j = 0; j < NKT; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[4 * j + i] = s[rt][j][i];
    // The lane's own maximum decides whether any row can have grown; only
    // then are the four lanes of each row reduced (a row's maximum grows
    // past the threshold only if one of its lanes' maxima does).
    const float lane_mx = lane_max<4 * NKT>(sv) * scale_log2;
    if (__builtin_amdgcn_ballot_w64(lane_mx > st.m_run[rt] + kRescaleLog2) != 0) {
      const float mx = wave_max_across_groups(lane_mx);
      const bool grow = mx > st.m_run[rt] + kRescaleLog2;
      const float m_new = grow ? mx : st.m_run[rt];
      const float alpha = (grow && st.m_run[rt] != -INFINITY) ? __builtin_amdgcn_exp2f(st.m_run[rt] - m_new)
                                                              : (grow ? 0.f : 1.f);
      st.l_acc[rt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) st.o[rt][dt] *= alpha;
      st.m_run[rt] = m_new;
    }
  }
}

template <bool BF16, int RT, int NKT>
__device__ __forceinline__ void d128_exp(RowState<BF16, RT>& st, const f32x4 (&s)[RT][NKT], float scale_log2,
                                         uint32_t (&pk)[RT][NKT][2]) {
  typedef Mfma<BF16> M;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float neg_m = st.m_run[rt] == -INFINITY ? 0.f : -st.m_run[rt];
#pragma unroll
    for (int j = 0; j < NKT; ++j) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][j][0], scale_log2, neg_m));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][j][1], scale_log2, neg_m));
      const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][j][2], scale_log2, neg_m));
      const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][j][3], scale_log2, neg_m));
      pk[rt][j][0] = M::pack2(p0, p1);
      pk[rt][j][1] = M::pack2(p2, p3);
    }
  }
}

template <bool BF16, int RT, int NKT>
__device__ __forceinline__ void d128_pv(RowState<BF16, RT>& st, const uint32_t (&pk)[RT][NKT][2], const char* sb,
                                        int kb0, int grp, int r16) {
  typedef Mfma<BF16> M;
  typedef typename M::frag frag;
  const int e = r16 >> 2;
  const int q = r16 & 3;
  const char* vb = sb + kHalf128;
  if constexpr (NKT == 1) {
    // 16 keys: one half of a 32-key block, through the K=16 MFMA whose A and B
    // operands are exactly one transposing read and one packed score block.
    const int kk = kb0 >> 1;
    const int key0 = 32 * kk + 4 * grp + e;
    const char* vrow = vb + (key0 + 16 * (kb0 & 1)) * kRowBytes128 + ((q & 1) << 3);
    const int vsw = (key0 & 7) << 1;
    v4i16 pb[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) pb[rt] = __builtin_bit_cast(v4i16, uint2{pk[rt][0][0], pk[rt][0][1]});
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const v4i16 av = lds_read_tr16(vrow + (((2 * dt + (q >> 1)) ^ vsw) << 4));
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) st.o[rt][dt] = M::run16(av, pb[rt], st.o[rt][dt]);
    }
    const v4i16 ones = M::ones4();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) st.l_acc[rt] = M::run16(ones, pb[rt], st.l_acc[rt]);
  } else {
    frag pf[RT][NKT / 2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int h = 0; h < NKT / 2; ++h)
        pf[rt][h] = __builtin_bit_cast(frag, uint4{pk[rt][2 * h][0], pk[rt][2 * h][1], pk[rt][2 * h + 1][0],
                                                   pk[rt][2 * h + 1][1]});
#pragma unroll
    for (int h = 0; h < NKT / 2; ++h) {
      const int kk = (kb0 >> 1) + h;
      const int key0 = 32 * kk + 4 * grp + e;
      const char* vrow = vb + key0 * kRowBytes128 + ((q & 1) << 3);
      const int vsw = (key0 & 7) << 1;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const char* p0 = vrow + (((2 * dt + (q >> 1)) ^ vsw) << 4);
        const v4i16 lo = lds_read_tr16(p0);
        const v4i16 hi = lds_read_tr16(p0 + 16 * kRowBytes128);
        const frag av = __builtin_bit_cast(frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) st.o[rt][dt] = M::run(av, pf[rt][h], st.o[rt][dt]);
      }
      const frag ones = M::ones8();
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) st.l_acc[rt] = M::run(ones, pf[rt][h], st.l_acc[rt]);
    }
  }
}

template <bool BF16, int RT, int NKT, int MODE>
__device__ __forceinline__ void d128_softmax_pv(RowState<BF16, RT>& st, f32x4 (&s)[RT][NKT], const char* sb, int kb0,
                                                int t0, int kv_end, int col0, int mask_mode, float scale_log2,
                                                int grp, int r16) {
  uint32_t pk[RT][NKT][2];
  d128_rowmax<BF16, RT, NKT, MODE>(st, s, kb0, t0, kv_end, col0, mask_mode, scale_log2, grp);
  d128_exp<BF16, RT, NKT>(st, s, scale_log2, pk);
  d128_pv<BF16, RT, NKT>(st, pk, sb, kb0, grp, r16);
}

// One pipelined step: the softmax of tile t (scores s_cur, stage sb) with the
// score MFMAs of tile t+1 (stage sb_next) between its exp and its P.V, all in
// one basic block after the row maxima.
template <bool BF16, int RT, int NKT, int MODE>
__device__ __forceinline__ void d128_pipe_step(RowState<BF16, RT>& st, f32x4 (&s_cur)[RT][NKT],
                                               f32x4 (&s_nxt)[RT][NKT], const char* sb, const char* sb_next, int kb0,
                                               int t0, int kv_end, int col0, int mask_mode, float scale_log2,
                                               int grp, int r16) {
  uint32_t pk[RT][NKT][2];
  d128_rowmax<BF16, RT, NKT, MODE>(st, s_cur, kb0, t0, kv_end, col0, mask_mode, scale_log2, grp);
  d128_exp<BF16, RT, NKT>(st, s_cur, scale_log2, pk);
  d128_scores<BF16, RT, NKT>(st, sb_next, kb0, grp, r16, s_nxt);
  d128_pv<BF16, RT, NKT>(st, pk, sb, kb0, grp, r16);
}

// Row bookkeeping, tree masks and softmax state of row tiles tile0 +
// tstride*rt (the queries arrive through LDS, see d128_read_q).
template <bool BF16, int RT>
__device__ __forceinline__ void d128_load_rows(RowState<BF16, RT>& st, const AttnArgs& a, const atlas_attn_work_t& w,
                                               const ItemCtx& c, int tile0, int tstride, int lane) {
  typedef typename Mfma<BF16>::frag frag;
  const int grp = lane >> 4;
  const int r16 = lane & 15;
  const int G = a.group;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int lr = (tile0 + tstride * rt) * 16 + r16;
    st.lrow[rt] = lr;
    st.row_ok[rt] = lr < w.num_rows;
    const int prow = w.row_start + (st.row_ok[rt] ? lr : 0);
    st.node_of[rt] = prow / G;
    st.head_of[rt] = w.kv_head * G + (prow - st.node_of[rt] * G);
    st.m_run[rt] = -INFINITY;
    st.l_acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) st.o[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.tbits[rt] = 0ull;
    st.climit[rt] = c.kv_len - c.qo_len + st.node_of[rt];
  }
  if (a.rope_cos != nullptr) {
    // Issued ahead of the page windows: ring_begin's wait covers both.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int64_t off = int64_t(c.qo_start + st.node_of[rt]) * a.rope_stride_token * 2;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        st.rcos[rt][ks] = *reinterpret_cast<const u32x4v*>(a.rope_cos + off + (ks * 4 + grp) * 16);
        st.rsin[rt][ks] = *reinterpret_cast<const u32x4v*>(a.rope_sin + off + (ks * 4 + grp) * 16);
      }
    }
  }
}

// The rows' tree ancestor words.  Loaded after the ring's first tiles are
// issued: they are needed only by the masked tiles at the end of a split, and
// loading them before would put a round trip ahead of the first KV tile.
template <bool BF16, int RT>
__device__ __forceinline__ void d128_load_masks(RowState<BF16, RT>& st, const AttnArgs& a, const ItemCtx& c) {
  if (a.mask_mode != ATLAS_MASK_TREE || a.mask_words != 1) return;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    st.tbits[rt] = st.row_ok[rt] ? a.tree_mask[c.qo_start + st.node_of[rt]] : 0ull;
}

// The mask column start a masked tile at t0 is tested against: the request's
// for one-word masks; for wide masks the tile's own start, after the rows'
// words of that tile are loaded.  (A wide tree is the rare case: the load
// waits for the loads in flight, the ring's included.)
template <bool BF16, int RT>
__device__ __forceinline__ int d128_tile_mask(RowState<BF16, RT>& st, const AttnArgs& a, const ItemCtx& c, int t0) {
  if (a.mask_mode != ATLAS_MASK_TREE || a.mask_words == 1) return c.col0;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    st.tbits[rt] = st.row_ok[rt] ? tile_mask_word(a, int64_t(c.qo_start + st.node_of[rt]), t0, c.col0) : 0ull;
  return t0;
}

// Queries of the wave's rows from the LDS staging area into registers (rows
// past num_rows are zeroed), rotated when the step carries RoPE tables.  Runs
// right after the first ring step: stage 3 is overwritten only after the next
// barrier.
template <bool BF16, int RT>
__device__ __forceinline__ void d128_read_q(RowState<BF16, RT>& st, const char* lds, bool rope, int lane) {
  typedef typename Mfma<BF16>::frag frag;
  const int grp = lane >> 4;
  const int r16 = lane & 15;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const char* qrow = lds + kQOffset + st.lrow[rt] * 256;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint4 v = *reinterpret_cast<const uint4*>(qrow + (((ks * 4 + grp) ^ r16) << 4));
      if (!st.row_ok[rt]) v = uint4{0, 0, 0, 0};
      st.qf[rt][ks] = __builtin_bit_cast(frag, v);
    }
  }
  if (rope) {
    // Granules ks and ks + 2 hold dims d and d + D/2: each other's partners.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const u32x4v lo = __builtin_bit_cast(u32x4v, st.qf[rt][ks]);
        const u32x4v hi = __builtin_bit_cast(u32x4v, st.qf[rt][ks + 2]);
        st.qf[rt][ks] = __builtin_bit_cast(frag, rope8<BF16>(lo, hi, st.rcos[rt][ks], st.rsin[rt][ks], true));
        st.qf[rt][ks + 2] =
            __builtin_bit_cast(frag, rope8<BF16>(hi, lo, st.rcos[rt][ks + 2], st.rsin[rt][ks + 2], false));
      }
  }
}

// The tile loop of one wave: RT row tiles over key blocks kb0 .. kb0+NKT-1 of
// every tile.  PIPE computes tile t+1's scores while tile t's softmax and P.V
// run (RT = 1, whole tiles); otherwise each tile is computed before its ring
// step.
template <bool BF16, int NL, int RT, int NKT, bool PIPE>
__device__ __forceinline__ void d128_loop(RowState<BF16, RT>& st, Ring<NL>& r, const AttnArgs& a, const ItemCtx& c,
                                          const char* lds, int kb0, int lane) {
  const int grp = lane >> 4;
  const int r16 = lane & 15;
  const int nt = r.nt;
  if (nt <= 0) return;
  ring_first<NL>(r);
  d128_read_q<BF16, RT>(st, lds, a.rope_cos != nullptr, lane);
  if constexpr (PIPE) {
    f32x4 s_cur[RT][NKT];
    f32x4 s_nxt[RT][NKT];
    d128_scores<BF16, RT, NKT>(st, lds, kb0, grp, r16, s_cur);
    const int n_pipe = nt - 1;
    const int plain_end = min(c.nt_plain, n_pipe);
    int t = 0;
    for (; t < plain_end; ++t) {
      ring_step<NL>(r, t);
      d128_pipe_step<BF16, RT, NKT, kPlain>(st, s_cur, s_nxt, lds + (t % kStages128) * kTile128,
                                            lds + ((t + 1) % kStages128) * kTile128, kb0, c.t_first + t * kTileKeys,
                                            c.kv_end, c.col0, a.mask_mode, a.scale_log2, grp, r16);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < NKT; ++j) s_cur[rt][j] = s_nxt[rt][j];
    }
    for (; t < n_pipe; ++t) {
      ring_step<NL>(r, t);
      const int t0 = c.t_first + t * kTileKeys;
      const int col0_t = d128_tile_mask<BF16, RT>(st, a, c, t0);
      d128_pipe_step<BF16, RT, NKT, kMasked>(st, s_cur, s_nxt, lds + (t % kStages128) * kTile128,
                                             lds + ((t + 1) % kStages128) * kTile128, kb0, t0,
                                             c.kv_end, col0_t, a.mask_mode, a.scale_log2, grp, r16);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < NKT; ++j) s_cur[rt][j] = s_nxt[rt][j];
    }
    ring_step<NL>(r, t);
    if (t < c.nt_plain)
      d128_softmax_pv<BF16, RT, NKT, kPlain>(st, s_cur, lds + (t % kStages128) * kTile128, kb0,
                                            c.t_first + t * kTileKeys, c.kv_end, c.col0, a.mask_mode, a.scale_log2,
                                            grp, r16);
    else
      d128_softmax_pv<BF16, RT, NKT, kMasked>(st, s_cur, lds + (t % kStages128) * kTile128, kb0,
                                           c.t_first + t * kTileKeys, c.kv_end,
                                           d128_tile_mask<BF16, RT>(st, a, c, c.t_first + t * kTileKeys),
                                           a.mask_mode, a.scale_log2, grp, r16);
  } else {
    f32x4 s[RT][NKT];
    int t = 0;
    for (; t < c.nt_plain; ++t) {
      const char* sb = lds + (t % kStages128) * kTile128;
      d128_scores<BF16, RT, NKT>(st, sb, kb0, grp, r16, s);
      d128_softmax_pv<BF16, RT, NKT, kPlain>(st, s, sb, kb0, c.t_first + t * kTileKeys, c.kv_end, c.col0,
                                            a.mask_mode, a.scale_log2, grp, r16);
      ring_step<NL>(r, t);
    }
    for (; t < nt; ++t) {
      const char* sb = lds + (t % kStages128) * kTile128;
      const int t0 = c.t_first + t * kTileKeys;
      const int col0_t = d128_tile_mask<BF16, RT>(st, a, c, t0);
      d128_scores<BF16, RT, NKT>(st, sb, kb0, grp, r16, s);
      d128_softmax_pv<BF16, RT, NKT, kMasked>(st, s, sb, kb0, t0, c.kv_end, col0_t,
                                           a.mask_mode, a.scale_log2, grp, r16);
      ring_step<NL>(r, t);
    }
  }
}

// Writes one finished row (the final output, or the split's partial state,
// both in the output dtype) for the lanes' D columns 16*dt + 4*grp .. +3, dt
// in [dt0, dt0 + NDT).
template <bool BF16, int NDT>
__device__ __forceinline__ void d128_store(const AttnArgs& a, const atlas_attn_work_t& w, const ItemCtx& c, int node,
                                           int head, int lrow, bool row_ok, const f32x4 (&o)[NDT], int dt0,
                                           float inv, float lse2, bool write_lse, int grp) {
  typedef Mfma<BF16> M;
  constexpr int D = 128;
  if (!row_ok) return;
  const bool final_row = w.partial_row < 0;
  const int64_t prow = int64_t(w.partial_row) + lrow;
  if (!final_row && prow >= a.part_rows) return;
  char* orow = final_row ? a.out + ((int64_t(c.qo_start + node) * a.out_stride_token +
                                     int64_t(head) * a.out_stride_head) * 2)
                         : reinterpret_cast<char*>(a.part_o + prow * D);
  // Split partial rows are written through to memory (agent-scope stores):
  // the merge launch reads them from other XCDs, and nothing of them is left
  // dirty in this XCD's L2 at the end of the launch (0.3 us per layer less
  // on the 16k forest).
#pragma unroll
  for (int i = 0; i < NDT; ++i) {
    const int dt = dt0 + i;
    const uint32_t lo = uint32_t(M::from_float(o[i][0] * inv)) | (uint32_t(M::from_float(o[i][1] * inv)) << 16);
    const uint32_t hi = uint32_t(M::from_float(o[i][2] * inv)) | (uint32_t(M::from_float(o[i][3] * inv)) << 16);
    char* dst = orow + (dt * 16 + grp * 4) * 2;
    if (final_row)
      *reinterpret_cast<uint2*>(dst) = uint2{lo, hi};
    else
      __hip_atomic_store(reinterpret_cast<uint64_t*>(dst), uint64_t(lo) | (uint64_t(hi) << 32), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  if (write_lse && grp == 0) {
    if (!final_row) __hip_atomic_store(a.part_lse + prow, lse2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else if (a.lse != nullptr) a.lse[int64_t(c.qo_start + node) * a.num_qo_heads + head] = lse2 * kLn2;
  }
}

// Whole row tiles: normalise and store.
template <bool BF16, int RT>
__device__ __forceinline__ void d128_store_rows(RowState<BF16, RT>& st, const AttnArgs& a,
                                                const atlas_attn_work_t& w, const ItemCtx& c, int lane) {
  const int grp = lane >> 4;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float l_tot = st.l_acc[rt][0];
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const float lse2 = l_tot > 0.f ? st.m_run[rt] + __builtin_log2f(l_tot) : -INFINITY;
    d128_store<BF16, 8>(a, w, c, st.node_of[rt], st.head_of[rt], st.lrow[rt], st.row_ok[rt], st.o[rt], 0, inv, lse2,
                        true, grp);
  }
}

// Key parts of one row tile held by S waves (part index p, LDS slot base j0 of
// the tile's first part): each part's unnormalised O, running max and row sum
// go to LDS; after a workgroup barrier, part p combines the S states for D
// columns [128 p / S, 128 (p + 1) / S) and stores them.  The caller's barriers
// bracket the LDS exchange (every wave of the workgroup takes part in them).
constexpr int kPartBytes = 8 * 64 * 16 + 2 * 64 * 4;  // O^T accumulators, then m and l per lane

template <bool BF16>
__device__ __forceinline__ void d128_part_put(const RowState<BF16, 1>& st, char* lds, int slot, int lane) {
  char* base = lds + slot * kPartBytes;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(base + (dt * 64 + lane) * 16) = st.o[0][dt];
  reinterpret_cast<float*>(base + 8 * 64 * 16)[lane] = st.m_run[0];
  reinterpret_cast<float*>(base + 8 * 64 * 16)[64 + lane] = st.l_acc[0][0];
}

template <bool BF16, int S>
__device__ __forceinline__ void d128_part_merge(const RowState<BF16, 1>& st, const char* lds, int slot0, int p,
                                                const AttnArgs& a, const atlas_attn_work_t& w, const ItemCtx& c,
                                                int lane) {
  constexpr int NDT = 8 / S;
  float m[S], l[S];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const float* ml = reinterpret_cast<const float*>(lds + (slot0 + i) * kPartBytes + 8 * 64 * 16);
    m[i] = ml[lane];
    l[i] = ml[64 + lane];
    mx = fmaxf(mx, m[i]);
  }
  float wsum = 0.f;
  float wt[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    wt[i] = m[i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[i] - mx);
    wsum += wt[i] * l[i];
  }
  f32x4 o[NDT];
#pragma unroll
  for (int k = 0; k < NDT; ++k) {
    const int dt = p * NDT + k;
    o[k] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < S; ++i)
      o[k] += wt[i] * *reinterpret_cast<const f32x4*>(lds + (slot0 + i) * kPartBytes + (dt * 64 + lane) * 16);
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const float lse2 = wsum > 0.f ? mx + __builtin_log2f(wsum) : -INFINITY;
  d128_store<BF16, NDT>(a, w, c, st.node_of[0], st.head_of[0], st.lrow[0], st.row_ok[0], o, p * NDT, inv, lse2,
                        p == 0, lane >> 4);
}

// Row tiles of an item whose count T = 4k + R with k <= 2 and R in {1, 2}:
// waves 0..3 (one per SIMD) own whole tiles w and w + 4 (k per wave); the R
// leftover tiles are split by keys over waves 4..7 (R = 1: four 16-key
// quarters of every tile; R = 2: two 32-key halves per tile).  Every SIMD
// then carries k + R/4 tile-units instead of the k + 1 (or more) of one tile
// per wave.  All eight waves issue KV loads: with four loaders the paged
// stream alone runs at two thirds of the eight-loader rate.
template <bool BF16, int NL>
__device__ __forceinline__ void d128_item_split(const AttnArgs& a, const atlas_attn_work_t& w, const ItemCtx& c,
                                                char* lds, Ring<NL>& r, int T, int wave, int lane) {
  const int R = T & 3;
  const int k = T >> 2;
  if (wave < 4) {
    if (k == 2) {
      RowState<BF16, 2> st;
      d128_load_rows<BF16, 2>(st, a, w, c, wave, 4, lane);
      ring_begin<NL>(r, a, w, c, T);
      d128_load_masks<BF16, 2>(st, a, c);
      d128_loop<BF16, NL, 2, 4, false>(st, r, a, c, lds, 0, lane);
      d128_store_rows<BF16, 2>(st, a, w, c, lane);
    } else if (k == 1) {
      RowState<BF16, 1> st;
      d128_load_rows<BF16, 1>(st, a, w, c, wave, 4, lane);
      ring_begin<NL>(r, a, w, c, T);
      d128_load_masks<BF16, 1>(st, a, c);
      d128_loop<BF16, NL, 1, 4, true>(st, r, a, c, lds, 0, lane);
      d128_store_rows<BF16, 1>(st, a, w, c, lane);
    } else {
      ring_only<NL>(r, a, w, c, T);
    }
    bare_barrier();
    bare_barrier();
    return;
  }
  const int j = wave - 4;
  RowState<BF16, 1> st;
  if (R == 1) {
    d128_load_rows<BF16, 1>(st, a, w, c, 4 * k, 0, lane);
    ring_begin<NL>(r, a, w, c, T);
    d128_load_masks<BF16, 1>(st, a, c);
    d128_loop<BF16, NL, 1, 1, false>(st, r, a, c, lds, j, lane);
    bare_barrier();
    d128_part_put<BF16>(st, lds, j, lane);
    bare_barrier();
    d128_part_merge<BF16, 4>(st, lds, 0, j, a, w, c, lane);
  } else {
    d128_load_rows<BF16, 1>(st, a, w, c, 4 * k + (j >> 1), 0, lane);
    ring_begin<NL>(r, a, w, c, T);
    d128_load_masks<BF16, 1>(st, a, c);
    d128_loop<BF16, NL, 1, 2, false>(st, r, a, c, lds, 2 * (j & 1), lane);
    bare_barrier();
    d128_part_put<BF16>(st, lds, j, lane);
    bare_barrier();
    d128_part_merge<BF16, 2>(st, lds, j & ~1, j & 1, a, w, c, lane);
  }
}

// Other row counts: tile i on wave i % 8 (two per wave past 8 tiles); every
// wave loads its share of the KV.
template <bool BF16>
__device__ __forceinline__ void d128_item_rr(const AttnArgs& a, const atlas_attn_work_t& w, const ItemCtx& c,
                                             char* lds, Ring<8>& r, int T, int wave, int lane) {
  const int mine = (wave < T ? 1 : 0) + (wave + 8 < T ? 1 : 0);
  if (mine == 2) {
    RowState<BF16, 2> st;
    d128_load_rows<BF16, 2>(st, a, w, c, wave, 8, lane);
    ring_begin<8>(r, a, w, c, T);
    d128_load_masks<BF16, 2>(st, a, c);
    d128_loop<BF16, 8, 2, 4, false>(st, r, a, c, lds, 0, lane);
    d128_store_rows<BF16, 2>(st, a, w, c, lane);
  } else if (mine == 1) {
    RowState<BF16, 1> st;
    d128_load_rows<BF16, 1>(st, a, w, c, wave, 8, lane);
    ring_begin<8>(r, a, w, c, T);
    d128_load_masks<BF16, 1>(st, a, c);
    d128_loop<BF16, 8, 1, 4, true>(st, r, a, c, lds, 0, lane);
    d128_store_rows<BF16, 1>(st, a, w, c, lane);
  } else {
    ring_only<8>(r, a, w, c, T);
  }
}

template <int NL>
__device__ __forceinline__ void ring_init(Ring<NL>& r, const AttnArgs& a, const char* head_base, const int32_t* pages,
                                          const ItemCtx& c, int last_key, int li, int lane, uint32_t lds0) {
  r.head_base = head_base;
  r.pages = pages;
  r.page_stride = a.page_stride;
  r.token_stride = a.token_stride;
  r.v_offset = a.v_offset;
  r.page_size = a.page_size;
  r.page_shift = a.page_shift;
  r.t_first = c.t_first;
  r.nt = c.nt;
  r.last_key = last_key;
  r.page0 = c.t_first >> a.page_shift;
  r.last_page = max(last_key, 0) >> a.page_shift;
  r.win = 0;
  r.win_cur = 0;
  r.win_nxt = 0;
  r.li = li;
  r.lane = lane;
  r.lds0 = lds0;
  r.nt_full = c.nt - ((c.t_first + c.nt * kTileKeys - 1 > last_key) ? 1 : 0);
  static_assert(NL % 4 == 0, "block keys & 15 must not depend on the block's round j");
  const int c16p = lane & 15;
  const int kmask = min(a.page_size, kTileKeys) - 1;
#pragma unroll
  for (int j = 0; j < 16 / NL; ++j) {
    const int key = 4 * (NL * j + li) + (lane >> 4);
    const uint32_t row = uint32_t(key & kmask) * uint32_t(a.token_stride);
    r.off_k[j] = row + uint32_t((c16p ^ (key & 15)) << 4);
    r.off_v[j] = row + uint32_t((c16p ^ ((key & 7) << 1)) << 4);
  }
}

// Fused append: the request's newest qo_len tokens occupy its last qo_len key
// positions.  The rows of those positions that fall in this item's key range
// are copied, for this item's KV head, from the caller's K / V rows into the
// paged cache before any tile is loaded (the loads of the masked tail tile
// read them back).  32 lanes per position (16 granules of K, 16 of V), 16
// positions per pass; with RoPE tables the K granules are rotated on the way.  The planner gives every (request, KV head) a single row
// block, so no other workgroup reads these rows.
template <bool BF16>
__device__ __forceinline__ void d128_append_rows(const AttnArgs& a, const atlas_attn_work_t& w, const ItemCtx& c) {
  const int first_new = c.kv_len - c.qo_len;
  const int a0 = max(c.t_first, first_new);
  const int a1 = c.kv_end;
  const int tid = threadIdx.x;
  const int g = tid & 15;
  const bool is_v = (tid >> 4) & 1;
  for (int p = a0 + (tid >> 5); p < a1; p += 16) {
    const int node = p - first_new;
    const char* src = (is_v ? a.app_v : a.app_k) +
                      (int64_t(c.qo_start + node) * a.app_stride_token + int64_t(w.kv_head) * a.app_stride_head) * 2;
    const int32_t pid = a.kv_indices[int64_t(w.page_offset) + (p >> a.page_shift)];
    char* dst = const_cast<char*>(a.kv) + int64_t(pid) * a.page_stride + int64_t(p & (a.page_size - 1)) * a.token_stride +
                (is_v ? a.v_offset : 0) + int64_t(w.kv_head) * a.head_stride;
    u32x4v v = *reinterpret_cast<const u32x4v*>(src + g * 16);
    if (a.rope_cos != nullptr && !is_v) {
      const int64_t off = int64_t(c.qo_start + node) * a.rope_stride_token * 2 + g * 16;
      const u32x4v partner = *reinterpret_cast<const u32x4v*>(src + (g ^ 8) * 16);
      v = rope8<BF16>(v, partner, *reinterpret_cast<const u32x4v*>(a.rope_cos + off),
                      *reinterpret_cast<const u32x4v*>(a.rope_sin + off), g < 8);
    }
    *reinterpret_cast<u32x4v*>(dst + g * 16) = v;
  }
}

// 8 waves (two per SIMD), one workgroup per CU.  The item's row-tile count
// picks the wave layout (d128_item_split / d128_item_rr).
template <bool BF16>
__global__ __launch_bounds__(512, 1) void tree_attn_d128_kernel(AttnArgs a) {
  constexpr int D = 128;
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes128];

  const int lane = threadIdx.x & 63;
  // The item's first page-id window depends only on the workgroup index, so
  // it is requested before (and travels with) the work item.
  const int win0 = a.page_window != nullptr ? a.page_window[int64_t(blockIdx.x) * 64 + lane] : 0;
  const atlas_attn_work_t w = a.work[blockIdx.x];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  ItemCtx c;
  c.win0 = win0;
  c.qo_start = w.qo_start;
  c.qo_len = w.qo_len;
  c.kv_len = w.kv_len;
  c.kv_end = min(w.kv_end, c.kv_len);

  int vis_all = c.kv_end;
  c.col0 = 0;
  if (a.mask_mode == ATLAS_MASK_TREE) {
    c.col0 = w.mask_col_start;
    vis_all = min(vis_all, c.col0);
  } else if (a.mask_mode == ATLAS_MASK_CAUSAL) {
    vis_all = min(vis_all, c.kv_len - c.qo_len + 1);
  }

  c.t_first = __builtin_amdgcn_readfirstlane(w.kv_start < c.kv_end ? w.kv_start : c.kv_end);
  c.nt = __builtin_amdgcn_readfirstlane((c.kv_end - c.t_first + kTileKeys - 1) / kTileKeys);
  // Leading tiles wholly below vis_all need no mask.
  c.nt_plain = __builtin_amdgcn_readfirstlane(
      min(c.nt, vis_all >= c.t_first + kTileKeys ? (vis_all - c.t_first) / kTileKeys : 0));
  const int last_key = __builtin_amdgcn_readfirstlane(c.kv_end - 1);
  const char* head_base = a.kv + int64_t(w.kv_head) * a.head_stride;
  const int32_t* pages = a.kv_indices + w.page_offset;
  const uint32_t lds0 = lds_offset(lds);
  if (a.app_k != nullptr && max(c.t_first, c.kv_len - c.qo_len) < c.kv_end) {
    // every wave's stores are acknowledged before any wave issues a load
    d128_append_rows<BF16>(a, w, c);
    wait_vmcnt<0>();
    bare_barrier();
  }

  const int T = __builtin_amdgcn_readfirstlane((w.num_rows + 15) / 16);
  const int R = T & 3;
  if (T <= 10 && (R == 1 || R == 2)) {
    Ring<8> r;
    ring_init<8>(r, a, head_base, pages, c, last_key, wave, lane, lds0);
    d128_item_split<BF16, 8>(a, w, c, lds, r, T, wave, lane);
  } else {
    Ring<8> r;
    ring_init<8>(r, a, head_base, pages, c, last_key, wave, lane, lds0);
    d128_item_rr<BF16>(a, w, c, lds, r, T, wave, lane);
  }
}


// Work-shape choice: the fewest (compute waves x row tiles) slots that cover
// the row tiles, preferring more waves (fewer tiles per wave).
inline void choose_shape(int row_tiles, int& nwc, int& rt) {
  int best = 1 << 30;
  nwc = 4;
  rt = 3;
  for (int r = 1; r <= 3; ++r) {
    for (int nw = 1; nw <= kWaves; ++nw) {
      if (nw * r < row_tiles) continue;
      const int slots = nw * r;
      if (slots < best || (slots == best && r < rt)) {
        best = slots;
        nwc = nw;
        rt = r;
      }
    }
  }
}

template <int D, bool BF16, int RT, int NWC>
void launch_shape(const AttnArgs& args, int num_work, hipStream_t stream) {
  hipLaunchKernelGGL((tree_attn_kernel<D, BF16, RT, NWC>), dim3(num_work), dim3(kThreads), 0, stream, args);
}

// head_dim 128 with power-of-two pages of >= 16 tokens: KV streamed by
// direct-to-LDS loads through a 4-tile ring (one workgroup of 8 waves per
// CU, two waves per SIMD), up to 16 row tiles per item.
template <bool BF16>
bool launch_d128(const AttnArgs& args, int num_work, int row_tiles, hipStream_t stream) {
  if (row_tiles > 16) return false;
  hipLaunchKernelGGL((tree_attn_d128_kernel<BF16>), dim3(num_work), dim3(512), 0, stream, args);
  return true;
}

template <int D, bool BF16>
int launch_attn(const AttnArgs& args, int num_work, int row_tiles, const MergeArgs& margs, int num_merge,
                int max_rows, hipStream_t stream) {
  int rc;
  int nwc, rt;
  if constexpr (D == 128) {
    if (args.page_shift >= 4) {
      if (!launch_d128<BF16>(args, num_work, row_tiles, stream)) {
        set_error("no kernel shape for %d row tiles", row_tiles);
        return ATLAS_EUNSUPPORTED;
      }
      if ((rc = launch_status("tree_attn_d128_kernel"))) return rc;
      goto merge;
    }
  }
  choose_shape(row_tiles, nwc, rt);
  if (row_tiles > 3 * kWaves) {
    set_error("no kernel shape for %d row tiles", row_tiles);
    return ATLAS_EUNSUPPORTED;
  }
  switch (rt * 10 + nwc) {
    case 11: launch_shape<D, BF16, 1, 1>(args, num_work, stream); break;
    case 12: launch_shape<D, BF16, 1, 2>(args, num_work, stream); break;
    case 13: launch_shape<D, BF16, 1, 3>(args, num_work, stream); break;
    case 14: launch_shape<D, BF16, 1, 4>(args, num_work, stream); break;
    case 22: launch_shape<D, BF16, 2, 2>(args, num_work, stream); break;
    case 23: launch_shape<D, BF16, 2, 3>(args, num_work, stream); break;
    case 24: launch_shape<D, BF16, 2, 4>(args, num_work, stream); break;
    case 33: launch_shape<D, BF16, 3, 3>(args, num_work, stream); break;
    case 34: launch_shape<D, BF16, 3, 4>(args, num_work, stream); break;
    default:
      set_error("no kernel shape for %d row tiles (rt=%d, waves=%d)", row_tiles, rt, nwc);
      return ATLAS_EUNSUPPORTED;
  }
  if ((rc = launch_status("tree_attn_kernel"))) return rc;
merge:
  if (num_merge > 0) {
    const dim3 grid(num_merge, (max_rows + kMergeRowsPerBlock - 1) / kMergeRowsPerBlock);
    hipLaunchKernelGGL((tree_attn_merge_kernel<D, BF16>), grid, dim3(kMergeThreads), 0, stream, margs);
    if ((rc = launch_status("tree_attn_merge_kernel"))) return rc;
  }
  return ATLAS_OK;
}

}  // namespace
}  // namespace atlas

namespace atlas {
namespace {

// Plan-time page-id windows: lane l of item i receives the id of the item's
// page (first page + l), clamped to the item's last page, exactly the window
// the head_dim-128 kernel would otherwise read after loading the work item.
__global__ __launch_bounds__(64) void attn_page_windows_kernel(const atlas_attn_work_t* work,
                                                               const int32_t* kv_indices, int page_shift,
                                                               int32_t* window) {
  const atlas_attn_work_t w = work[blockIdx.x];
  const int l = threadIdx.x;
  const int kv_end = min(w.kv_end, w.kv_len);
  const int t_first = w.kv_start < kv_end ? w.kv_start : kv_end;
  int id = 0;
  if (t_first < kv_end) {
    const int page0 = t_first >> page_shift;
    const int last_page = (kv_end - 1) >> page_shift;
    id = kv_indices[int64_t(w.page_offset) + min(page0 + l, last_page)];
  }
  window[int64_t(blockIdx.x) * 64 + l] = id;
}

// A plan's device set-up in one launch: blocks [0, num_work) write the page
// windows (as attn_page_windows_kernel, reading the caller's page table), the
// blocks after them copy the page table and the tree mask words into the
// plan's own buffers.
__global__ __launch_bounds__(64) void attn_plan_install_kernel(const atlas_attn_work_t* work, int num_work,
                                                               const int32_t* src_indices, int64_t n_indices,
                                                               int32_t* dst_indices, const int64_t* src_words,
                                                               int64_t n_words, int64_t* dst_words, int page_shift,
                                                               int32_t* window) {
  if (int(blockIdx.x) < num_work) {
    const atlas_attn_work_t w = work[blockIdx.x];
    const int l = threadIdx.x;
    const int kv_end = min(w.kv_end, w.kv_len);
    const int t_first = w.kv_start < kv_end ? w.kv_start : kv_end;
    int id = 0;
    if (t_first < kv_end) {
      const int page0 = t_first >> page_shift;
      const int last_page = (kv_end - 1) >> page_shift;
      id = src_indices[int64_t(w.page_offset) + min(page0 + l, last_page)];
    }
    window[int64_t(blockIdx.x) * 64 + l] = id;
    return;
  }
  const int64_t stride = int64_t(gridDim.x - num_work) * 64;
  const int64_t t = int64_t(blockIdx.x - num_work) * 64 + threadIdx.x;
  for (int64_t i = t; i < n_indices; i += stride) dst_indices[i] = src_indices[i];
  for (int64_t i = t; i < n_words; i += stride) dst_words[i] = src_words[i];
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" int atlas_attn_plan_install(const atlas_attn_work_t* work_dev, int num_work,
                                       const int32_t* src_indices_dev, int64_t n_indices, int32_t* dst_indices_dev,
                                       const int64_t* src_words_dev, int64_t n_words, int64_t* dst_words_dev,
                                       int page_size, int32_t* window_dev, void* stream) {
  ATLAS_REQUIRE(num_work >= 0 && n_indices >= 0 && n_words >= 0, "negative count");
  ATLAS_REQUIRE(n_indices == 0 || (src_indices_dev && dst_indices_dev), "page table buffers must not be NULL");
  ATLAS_REQUIRE(n_words == 0 || (src_words_dev && dst_words_dev), "mask word buffers must not be NULL");
  const int windows = window_dev != nullptr ? num_work : 0;
  if (windows) {
    ATLAS_REQUIRE(work_dev && src_indices_dev, "windows need the work list and the page table");
    ATLAS_REQUIRE(page_size > 0 && (page_size & (page_size - 1)) == 0, "page_size must be a power of two, got %d",
                  page_size);
  }
  const int64_t most = n_indices > n_words ? n_indices : n_words;
  const int copy_blocks = most > 0 ? static_cast<int>(std::min<int64_t>((most + 255) / 256, 256)) : 0;
  if (windows + copy_blocks == 0) return ATLAS_OK;
  const int shift = page_size > 0 ? __builtin_ctz(static_cast<unsigned>(page_size)) : 0;
  hipLaunchKernelGGL(attn_plan_install_kernel, dim3(windows + copy_blocks), dim3(64), 0,
                     static_cast<hipStream_t>(stream), work_dev, windows, src_indices_dev, n_indices, dst_indices_dev,
                     src_words_dev, n_words, dst_words_dev, shift, window_dev);
  return launch_status("attn_plan_install_kernel");
}

extern "C" int atlas_attn_page_windows(const atlas_attn_work_t* work_dev, int num_work,
                                       const int32_t* kv_indices_dev, int page_size, int32_t* window_dev,
                                       void* stream) {
  ATLAS_REQUIRE(num_work >= 0, "negative work count");
  if (num_work == 0) return ATLAS_OK;
  ATLAS_REQUIRE(work_dev && kv_indices_dev && window_dev, "work, kv_indices and window must not be NULL");
  ATLAS_REQUIRE(page_size > 0 && (page_size & (page_size - 1)) == 0, "page_size must be a power of two, got %d",
                page_size);
  const int shift = __builtin_ctz(static_cast<unsigned>(page_size));
  hipLaunchKernelGGL(attn_page_windows_kernel, dim3(num_work), dim3(64), 0, static_cast<hipStream_t>(stream),
                     work_dev, kv_indices_dev, shift, window_dev);
  return launch_status("attn_page_windows_kernel");
}

namespace {
int current_device_scratch(void** out);
}

// use_scratch: the split partial states go to the library's device scratch
// array (workspace_dev is ignored, workspace_bytes gives the rows in use);
// its address is looked up only after every argument has been checked.
static int verify_attn_impl(bool use_scratch,
    const void* q, int64_t q_stride_token, int64_t q_stride_head, const void* kv_cache,
    int64_t page_stride, int64_t kv_v_offset, int64_t token_stride, int64_t kv_head_stride,
    const int32_t* qo_indptr_dev,
    const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev, const int32_t* kv_len_dev,
    int mask_mode, const uint64_t* tree_mask_dev, const int32_t* mask_col_start_dev, int tree_mask_words,
    const atlas_attn_work_t* work_dev, int num_work, const int32_t* page_window_dev,
    const atlas_attn_merge_t* merge_dev, int num_merge, int64_t merge_partial_rows, int max_rows_per_item,
    int num_qo_heads, int num_kv_heads, int head_dim,
    int page_size, float sm_scale, int dtype, void* out, int64_t out_stride_token,
    int64_t out_stride_head, float* lse, void* workspace_dev, size_t workspace_bytes,
    void* stream, const void* append_k, const void* append_v, int64_t append_stride_token,
    int64_t append_stride_head, const void* rope_cos, const void* rope_sin, int64_t rope_stride_token) {
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
  ATLAS_REQUIRE(mask_mode != ATLAS_MASK_TREE || tree_mask_words >= 1, "tree_mask_words must be >= 1, got %d",
                tree_mask_words);
  ATLAS_REQUIRE(num_work >= 0 && num_merge >= 0, "negative work counts");
  ATLAS_REQUIRE(max_rows_per_item > 0 && max_rows_per_item <= kMaxRowsPerItem,
                "max_rows_per_item %d out of range (1..%d)", max_rows_per_item, kMaxRowsPerItem);
  ATLAS_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15) == 0 && (reinterpret_cast<uintptr_t>(kv_cache) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & 7) == 0,
                "q / kv_cache must be 16-byte aligned and out 8-byte aligned");
  ATLAS_REQUIRE(q_stride_head % 8 == 0 && q_stride_token % 8 == 0 && out_stride_head % 4 == 0 &&
                    out_stride_token % 4 == 0,
                "q strides must be multiples of 8 elements and out strides multiples of 4");
  ATLAS_REQUIRE(page_stride % 16 == 0 && token_stride % 16 == 0 && kv_v_offset % 16 == 0,
                "kv strides must be multiples of 16 bytes");
  // (the head_dim-128 kernel keeps a row's offset inside its page, up to 63
  // token rows plus 256 bytes, in 32 bits)
  ATLAS_REQUIRE(token_stride > 0 && token_stride <= (int64_t(1) << 25), "token_stride %lld out of range",
                (long long)token_stride);
  ATLAS_REQUIRE(kv_head_stride >= int64_t(head_dim) * 2 && kv_head_stride % 16 == 0,
                "kv_head_stride %lld must be a multiple of 16 bytes covering a head's row", (long long)kv_head_stride);
  if (num_work == 0) return ATLAS_OK;
  ATLAS_REQUIRE(work_dev != nullptr, "work list must not be NULL");
  const int row_tiles = (max_rows_per_item + 15) / 16;

  AttnArgs args{};
  args.q = static_cast<const char*>(q);
  args.q_stride_token = q_stride_token;
  args.q_stride_head = q_stride_head;
  args.kv = static_cast<const char*>(kv_cache);
  args.page_stride = page_stride;
  args.v_offset = kv_v_offset;
  args.token_stride = token_stride;
  args.head_stride = kv_head_stride;
  args.qo_indptr = qo_indptr_dev;
  args.kv_indptr = kv_indptr_dev;
  args.kv_indices = kv_indices_dev;
  args.kv_len = kv_len_dev;
  args.tree_mask = tree_mask_dev;
  args.mask_col_start = mask_col_start_dev;
  args.work = work_dev;
  args.page_window = page_window_dev;
  args.out = static_cast<char*>(out);
  args.out_stride_token = out_stride_token;
  args.out_stride_head = out_stride_head;
  args.lse = lse;
  args.scale_log2 = sm_scale * kLog2e;
  args.mask_mode = mask_mode;
  args.mask_words = mask_mode == ATLAS_MASK_TREE ? tree_mask_words : 1;
  args.group = num_qo_heads / num_kv_heads;
  args.num_qo_heads = num_qo_heads;
  args.page_size = page_size;
  args.page_shift = ilog2_exact(page_size);
  args.app_k = static_cast<const char*>(append_k);
  args.app_v = static_cast<const char*>(append_v);
  args.app_stride_token = append_stride_token;
  args.app_stride_head = append_stride_head;
  args.rope_cos = static_cast<const char*>(rope_cos);
  args.rope_sin = static_cast<const char*>(rope_sin);
  args.rope_stride_token = rope_stride_token;

  MergeArgs margs{};
  if (num_merge > 0) {
    ATLAS_REQUIRE(merge_dev != nullptr, "merge list must not be NULL when num_merge > 0");
    ATLAS_REQUIRE(use_scratch || workspace_dev != nullptr, "workspace must not be NULL when num_merge > 0");
    // The planner places the partial O rows first and the partial LSE after
    // them: workspace = [partial_rows * D 16-bit values][partial_rows floats].
    const size_t row_bytes = size_t(head_dim) * 2 + 4;
    ATLAS_REQUIRE(workspace_bytes % row_bytes == 0, "workspace_bytes must be partial_rows * (2 * head_dim + 4)");
    const size_t partial_rows = workspace_bytes / row_bytes;
    ATLAS_REQUIRE(merge_partial_rows > 0 && size_t(merge_partial_rows) <= partial_rows,
                  "the merge items reference %lld partial rows but the workspace holds %zu",
                  (long long)merge_partial_rows, partial_rows);
    if (use_scratch) {
      const int rc = current_device_scratch(&workspace_dev);
      if (rc != ATLAS_OK) return rc;
    }
    ATLAS_REQUIRE((reinterpret_cast<uintptr_t>(workspace_dev) & 15) == 0, "workspace must be 16-byte aligned");
    args.part_o = static_cast<uint16_t*>(workspace_dev);
    args.part_lse = reinterpret_cast<float*>(args.part_o + partial_rows * head_dim);
    args.part_rows = int64_t(partial_rows);
    margs.part_rows = int64_t(partial_rows);
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
    return bf16 ? launch_attn<128, true>(args, num_work, row_tiles, margs, num_merge, max_rows_per_item, s)
                : launch_attn<128, false>(args, num_work, row_tiles, margs, num_merge, max_rows_per_item, s);
  return bf16 ? launch_attn<64, true>(args, num_work, row_tiles, margs, num_merge, max_rows_per_item, s)
              : launch_attn<64, false>(args, num_work, row_tiles, margs, num_merge, max_rows_per_item, s);
}

extern "C" int atlas_tree_verify_attn(
    const void* q, int64_t q_stride_token, int64_t q_stride_head, const void* kv_cache,
    int64_t page_stride, int64_t kv_v_offset, int64_t token_stride, int64_t kv_head_stride,
    const int32_t* qo_indptr_dev,
    const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev, const int32_t* kv_len_dev,
    int mask_mode, const uint64_t* tree_mask_dev, const int32_t* mask_col_start_dev, int tree_mask_words,
    const atlas_attn_work_t* work_dev, int num_work, const int32_t* page_window_dev,
    const atlas_attn_merge_t* merge_dev, int num_merge, int64_t merge_partial_rows, int max_rows_per_item,
    int num_qo_heads, int num_kv_heads, int head_dim,
    int page_size, float sm_scale, int dtype, void* out, int64_t out_stride_token,
    int64_t out_stride_head, float* lse, void* workspace_dev, size_t workspace_bytes,
    void* stream) {
  return verify_attn_impl(false, q, q_stride_token, q_stride_head, kv_cache, page_stride, kv_v_offset, token_stride,
                          kv_head_stride,
                          qo_indptr_dev, kv_indptr_dev, kv_indices_dev, kv_len_dev, mask_mode, tree_mask_dev,
                          mask_col_start_dev, tree_mask_words, work_dev, num_work, page_window_dev, merge_dev, num_merge,
                          merge_partial_rows, max_rows_per_item, num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale, dtype, out,
                          out_stride_token, out_stride_head, lse, workspace_dev, workspace_bytes, stream, nullptr,
                          nullptr, 0, 0, nullptr, nullptr, 0);
}

extern "C" int atlas_tree_verify_attn_append(
    const void* q, int64_t q_stride_token, int64_t q_stride_head, const void* kv_cache,
    int64_t page_stride, int64_t kv_v_offset, int64_t token_stride, int64_t kv_head_stride,
    const int32_t* qo_indptr_dev,
    const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev, const int32_t* kv_len_dev,
    int mask_mode, const uint64_t* tree_mask_dev, const int32_t* mask_col_start_dev, int tree_mask_words,
    const atlas_attn_work_t* work_dev, int num_work, const int32_t* page_window_dev,
    const atlas_attn_merge_t* merge_dev, int num_merge, int64_t merge_partial_rows, int max_rows_per_item,
    int num_qo_heads, int num_kv_heads, int head_dim,
    int page_size, float sm_scale, int dtype, void* out, int64_t out_stride_token,
    int64_t out_stride_head, float* lse, void* workspace_dev, size_t workspace_bytes,
    const void* append_k, const void* append_v, int64_t append_stride_token, int64_t append_stride_head,
    const void* rope_cos, const void* rope_sin, int64_t rope_stride_token, void* stream) {
  ATLAS_REQUIRE(append_k && append_v, "append_k and append_v must not be NULL");
  ATLAS_REQUIRE((rope_cos == nullptr) == (rope_sin == nullptr), "rope_cos and rope_sin go together");
  ATLAS_REQUIRE(rope_cos == nullptr || ((reinterpret_cast<uintptr_t>(rope_cos) & 15) == 0 &&
                                        (reinterpret_cast<uintptr_t>(rope_sin) & 15) == 0 && rope_stride_token % 8 == 0),
                "rope tables must be 16-byte aligned with a token stride that is a multiple of 8 elements");
  if (head_dim != 128 || page_size < 16 || (page_size & (page_size - 1)) != 0) {
    set_error("the fused append needs head_dim 128 and a power-of-two page_size >= 16");
    return ATLAS_EUNSUPPORTED;
  }
  ATLAS_REQUIRE((reinterpret_cast<uintptr_t>(append_k) & 15) == 0 && (reinterpret_cast<uintptr_t>(append_v) & 15) == 0,
                "append rows must be 16-byte aligned");
  ATLAS_REQUIRE(append_stride_token % 8 == 0 && append_stride_head % 8 == 0,
                "append strides must be multiples of 8 elements");
  return verify_attn_impl(false, q, q_stride_token, q_stride_head, kv_cache, page_stride, kv_v_offset, token_stride,
                          kv_head_stride,
                          qo_indptr_dev, kv_indptr_dev, kv_indices_dev, kv_len_dev, mask_mode, tree_mask_dev,
                          mask_col_start_dev, tree_mask_words, work_dev, num_work, page_window_dev, merge_dev, num_merge,
                          merge_partial_rows, max_rows_per_item, num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale, dtype, out,
                          out_stride_token, out_stride_head, lse, workspace_dev, workspace_bytes, stream, append_k,
                          append_v, append_stride_token, append_stride_head, rope_cos, rope_sin, rope_stride_token);
}

// ---------------------------------------------------------------------------
// Allocation-free verify attention.  The split-KV partial states live in a
// file-scope device array instead of a caller workspace: one copy per GPU,
// loaded with the code object and held until the process ends.  Its device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and only that address is ever handed to kernels: in host code the
// array's name is a host-side stand-in, not a device address.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[ATLAS_ATTN_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];

// Device address of the current device's scratch array.
int current_device_scratch(void** out) {
  int dev = -1;
  int rc = hip_status(hipGetDevice(&dev), "hipGetDevice");
  if (rc != ATLAS_OK) return rc;
  ATLAS_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "device %d beyond the %d scratch slots", dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (rc != ATLAS_OK) return rc;
    ATLAS_REQUIRE(p != nullptr, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ATLAS_OK;
}

}  // namespace

extern "C" int atlas_tree_verify_attn_noalloc(
    const void* q, int64_t q_stride_token, int64_t q_stride_head, const void* kv_cache,
    int64_t page_stride, int64_t kv_v_offset, int64_t token_stride, int64_t kv_head_stride,
    const int32_t* qo_indptr_dev,
    const int32_t* kv_indptr_dev, const int32_t* kv_indices_dev, const int32_t* kv_len_dev,
    int mask_mode, const uint64_t* tree_mask_dev, const int32_t* mask_col_start_dev, int tree_mask_words,
    const atlas_attn_work_t* work_dev, int num_work, const int32_t* page_window_dev,
    const atlas_attn_merge_t* merge_dev, int num_merge, int64_t merge_partial_rows, int max_rows_per_item,
    int num_qo_heads, int num_kv_heads, int head_dim, int page_size, float sm_scale, int dtype, void* out,
    int64_t out_stride_token, int64_t out_stride_head, float* lse, int64_t partial_rows, void* stream) {
  // every buffer and shape is checked before the device is touched
  ATLAS_REQUIRE(q && kv_cache && out, "q, kv_cache and out must not be NULL");
  ATLAS_REQUIRE(qo_indptr_dev && kv_indptr_dev && kv_indices_dev && kv_len_dev,
                "indptr / indices / kv_len arrays must not be NULL");
  ATLAS_REQUIRE(num_work == 0 || work_dev != nullptr, "work list must not be NULL");
  ATLAS_REQUIRE(num_merge == 0 || merge_dev != nullptr, "merge list must not be NULL when num_merge > 0");
  ATLAS_REQUIRE(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128, got %d", head_dim);
  ATLAS_REQUIRE(partial_rows >= 0, "negative partial_rows");
  const size_t row_bytes = size_t(head_dim) * 2 + 4;
  ATLAS_REQUIRE(size_t(partial_rows) <= size_t(ATLAS_ATTN_SCRATCH_BYTES) / row_bytes,
                "%lld partial rows of %zu bytes exceed the %d-byte device scratch (at most %zu rows at head_dim %d)",
                (long long)partial_rows, row_bytes, ATLAS_ATTN_SCRATCH_BYTES,
                size_t(ATLAS_ATTN_SCRATCH_BYTES) / row_bytes, head_dim);
  ATLAS_REQUIRE(num_merge == 0 || partial_rows > 0, "a split plan needs partial_rows > 0");
  ATLAS_REQUIRE(num_merge == 0 || (merge_partial_rows > 0 && merge_partial_rows <= partial_rows),
                "the merge items reference %lld partial rows but partial_rows is %lld",
                (long long)merge_partial_rows, (long long)partial_rows);
  return verify_attn_impl(true, q, q_stride_token, q_stride_head, kv_cache, page_stride, kv_v_offset, token_stride,
                          kv_head_stride,
                          qo_indptr_dev, kv_indptr_dev, kv_indices_dev, kv_len_dev, mask_mode, tree_mask_dev,
                          mask_col_start_dev, tree_mask_words, work_dev, num_work, page_window_dev, merge_dev, num_merge,
                          merge_partial_rows, max_rows_per_item, num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale, dtype, out,
                          out_stride_token, out_stride_head, lse, nullptr, size_t(partial_rows) * row_bytes,
                          stream, nullptr, nullptr, 0, 0, nullptr, nullptr, 0);
}
