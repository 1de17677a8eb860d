// QSA (Qwen Sparse Attention) decode path on gfx950.
//
// Three launches per decode step:
//   qsa_prep    per token: q/k RMS norm + partial rope, K/V page append, indexer
//               query, raw indexer key append, and the pooled key of any block
//               the token completes (reference/model.py:270-294, 345-363)
//   qsa_select  per query: block scores sum_h relu(q_h . k_j)/sqrt(d) over the
//               eligible blocks and the top budget/ratio of them, ties to the
//               lower index (reference/model.py:297-313)
//   qsa_attend  split-K paged GQA attention over the selected blocks plus the
//               query's tail block on bf16 MFMA, then a combine that applies the
//               sigmoid output gate (reference/model.py:365-382)
//
// Bit-exactness: the block scores feed a top-k whose result must match the
// reference exactly, so everything upstream of them (indexer query, pooled
// block keys) reproduces torch's CPU rounding: the block mean sums 16-row chunks
// in order and then the chunk sums in order, RMS norms reduce 128/256-wide rows
// the way torch's vectorised CPU sum does (see torch_row_sumsq), rsqrt is
// 1/sqrt, and every multiply and add of the rope is rounded separately.

#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int QSA_D = 256;     // attention head dim
constexpr int IDX_D = 128;     // indexer head dim
constexpr int PREP_NT = 256;

// column of page row `row` in a transposed V page: tokens of each 32-row group
// are stored in the order the PV MFMA's k index visits them
__host__ __device__ __forceinline__ int v_slot(int row) {
  const int t = row & 31;
  return (row & ~31) + 8 * ((t & 15) >> 2) + 4 * (t >> 4) + (t & 3);
}

// y = rope(round_T(rms_norm(x) * w)) for one row of `n` channels held in LDS
// by threads 0..n-1 (n <= blockDim). Rotates the first `rope` channels with the
// cos/sin row given. Returns the value of channel tid (0 for tid >= n).
template <typename T>
__device__ float norm_rope_row(float* s_x, float* s_y, float* s_scr, int n, const float* w, float eps,
                               int rope, const float* cs, const float* sn) {
  const int tid = threadIdx.x;
  const float ss = torch_row_sumsq(s_x, n, s_scr);
  const float rinv = rsqrt_rn(add_rn(div_rn(ss, (float)n), eps));
  float y = 0.f;
  if (tid < n) {
    y = Act<T>::round(mul_rn(mul_rn(s_x[tid], rinv), w[tid]));
    s_y[tid] = y;
  }
  __syncthreads();
  if (tid < rope) {
    const int half = rope / 2;
    const float rot = tid < half ? -s_y[tid + half] : s_y[tid - half];
    y = add_rn(mul_rn(y, cs[tid]), mul_rn(rot, sn[tid]));
  }
  return y;
}

// The indexer key of block j (reference/model.py:289-294): the float32 mean
// of its `ratio` raw keys (16-row chunks summed in order, then the chunk sums in
// order, then divided by the count, as torch's CPU mean reduces them), cast to
// the key dtype, RMS-normed with k_norm, and roped at the block's first
// position. Rows at or after `new0` come from `fresh` (row t - new0), earlier
// ones from `cache`. Called by a whole block; threads 0..127 own a channel.
template <typename T>
__device__ float pool_block(int j, int ratio, int rope, float eps, const float* k_norm, const float* cos,
                           const float* sin, const T* cache, const T* fresh, int new0, float* blocks, float* s_x,
                           float* s_y, float* s_scr) {
  const int tid = threadIdx.x;
  const int t0 = j * ratio;
  if (tid < IDX_D) {
    float total = 0.f;
    for (int c0 = 0; c0 < ratio; c0 += 16) {
      float acc = 0.f;
      const int c1 = min(c0 + 16, ratio);
      for (int i = c0; i < c1; ++i) {
        const int tok = t0 + i;
        const float v = tok >= new0 ? Act<T>::load(fresh, (long)(tok - new0) * IDX_D + tid)
                                    : Act<T>::load(cache, (long)tok * IDX_D + tid);
        acc = add_rn(acc, v);
      }
      total = c0 == 0 ? acc : add_rn(total, acc);
    }
    s_x[tid] = Act<T>::round(div_rn(total, (float)ratio));
  }
  const float y = norm_rope_row<T>(s_x, s_y, s_scr, IDX_D, k_norm, eps, rope, cos + (long)t0 * rope,
                                   sin + (long)t0 * rope);
  if (tid < IDX_D) blocks[(long)j * IDX_D + tid] = y;
  return y;
}

template <typename T>
struct PrepArgs {
  const T* qg; const T* k_new; const T* v_new; const T* iq; const T* ik;
  const float* q_norm; const float* k_norm; const float* iq_norm; const float* ik_norm;
  const float* cos; const float* sin;
  const int* positions; const int* page_table;
  uint16_t* k_pool; uint16_t* v_pool; T* raw_keys; float* block_keys;
  uint16_t* q_out; float* iq_out;
  int batch, seq, hq, hkv, rope, idx_heads, ratio, page_size, max_pages, max_ctx, max_blocks;
  float eps;
};

// Roles 0..Hq-1: attention query head `role` (RMS norm, rope, bf16 hi/lo).
// Roles Hq..Hq+Hkv-1: key/value head (norm + rope the key, append both).
template <typename T>
__device__ void prep_head(const PrepArgs<T>& A, int b, int s, int role) {
  __shared__ float s_x[QSA_D], s_y[QSA_D], s_scr[32];
  const int row = b * A.seq + s;
  const int tid = threadIdx.x;
  const int pos = A.positions[b] + s;
  const float* cs = A.cos + (long)pos * A.rope;
  const float* sn = A.sin + (long)pos * A.rope;
  if (role < A.hq) {
    if (!A.qg) return;
    const T* src = A.qg + ((long)row * A.hq + role) * (2 * QSA_D);
    s_x[tid] = Act<T>::load(src, tid);
    const float y = norm_rope_row<T>(s_x, s_y, s_scr, QSA_D, A.q_norm, A.eps, A.rope, cs, sn);
    // the attention MFMA takes q as bf16: keep it as hi + lo so the product
    // carries ~16 mantissa bits (rows [2 * row] hold hi, [2 * row + 1] lo)
    const uint16_t hi = f32_to_bf16(y);
    A.q_out[((long)(2 * row) * A.hq + role) * QSA_D + tid] = hi;
    A.q_out[((long)(2 * row + 1) * A.hq + role) * QSA_D + tid] = f32_to_bf16(y - bf16_to_f32(hi));
    return;
  }
  if (!A.k_new) return;
  const int g = role - A.hq;
  const long src = ((long)row * A.hkv + g) * QSA_D;
  s_x[tid] = Act<T>::load(A.k_new, src + tid);
  const float y = norm_rope_row<T>(s_x, s_y, s_scr, QSA_D, A.k_norm, A.eps, A.rope, cs, sn);
  const int page = A.page_table[(long)b * A.max_pages + pos / A.page_size];
  const int prow = pos % A.page_size;
  const long kbase = (((long)page * A.hkv + g) * A.page_size + prow) * QSA_D;
  A.k_pool[kbase + tid] = f32_to_bf16(y);
  const long vbase = (((long)page * A.hkv + g) * QSA_D + tid) * A.page_size + v_slot(prow);
  A.v_pool[vbase] = f32_to_bf16(Act<T>::load(A.v_new, src + tid));
}

template <typename T>
__global__ __launch_bounds__(PREP_NT) void qsa_prep_kernel(PrepArgs<T> A) {
  const int row = blockIdx.x;               // b * seq + s
  const int b = row / A.seq, s = row % A.seq;
  const int role = blockIdx.y;
  const int tid = threadIdx.x;
  const int pos0 = A.positions[b];
  const int pos = pos0 + s;
  const float* cs = A.cos + (long)pos * A.rope;
  const float* sn = A.sin + (long)pos * A.rope;

  __shared__ float s_x[QSA_D], s_y[QSA_D], s_scr[32];

  if (role < A.hq + A.hkv) {
    prep_head<T>(A, b, s, role);
    return;
  }
  if (role == A.hq + A.hkv) {
    // -------- indexer query heads, one after another
    for (int h = 0; h < A.idx_heads; ++h) {
      __syncthreads();
      if (tid < IDX_D) s_x[tid] = Act<T>::load(A.iq, ((long)row * A.idx_heads + h) * IDX_D + tid);
      const float y = norm_rope_row<T>(s_x, s_y, s_scr, IDX_D, A.iq_norm, A.eps, A.rope, cs, sn);
      if (tid < IDX_D) A.iq_out[((long)row * A.idx_heads + h) * IDX_D + tid] = y;
    }
    return;
  }
  // -------- raw indexer key append, and the pooled key of a completed block
  if (tid < IDX_D) A.raw_keys[((long)b * A.max_ctx + pos) * IDX_D + tid] = A.ik[(long)row * IDX_D + tid];
  if ((pos + 1) % A.ratio != 0) return;
  pool_block<T>(pos / A.ratio, A.ratio, A.rope, A.eps, A.ik_norm, A.cos, A.sin,
                A.raw_keys + (long)b * A.max_ctx * IDX_D, A.ik + (long)b * A.seq * IDX_D, pos0,
                A.block_keys + (long)b * A.max_blocks * IDX_D, s_x, s_y, s_scr);
}

template <typename T>
struct PoolArgs {
  const T* raw_keys; const float* k_norm; const float* cos; const float* sin; float* block_keys;
  int first_block, n_blocks, ratio, rope, max_ctx, max_blocks;
  float eps;
};

// pooled keys of blocks first_block .. first_block + n_blocks - 1 from the raw-key cache
template <typename T>
__global__ __launch_bounds__(IDX_D) void qsa_pool_kernel(PoolArgs<T> A) {
  const int j = A.first_block + blockIdx.x, b = blockIdx.y;
  __shared__ float s_x[IDX_D], s_y[IDX_D], s_scr[32];
  pool_block<T>(j, A.ratio, A.rope, A.eps, A.k_norm, A.cos, A.sin, A.raw_keys + (long)b * A.max_ctx * IDX_D,
                nullptr, 1 << 30, A.block_keys + (long)b * A.max_blocks * IDX_D, s_x, s_y, s_scr);
}

// ---------------------------------------------------------------------------
// selection
// ---------------------------------------------------------------------------
constexpr int SEL_NT = 256;
constexpr int SEL_MAX_BLOCKS = 4096;    // eligible blocks one query may score
constexpr int SEL_CHUNK = SEL_NT / 16 * 8;   // blocks scored per preloaded chunk (128)

__device__ __forceinline__ unsigned long long sel_key(float s, int j) {
  unsigned u = __float_as_uint(s);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);     // order-preserving
  return (static_cast<unsigned long long>(u) << 32) | static_cast<unsigned>(0x7fffffff - j);
}

// An attention work item: one 32-token group of one page, rows [lo, hi) visible.
// .x = physical pool row of the group's first token (page * P + row0),
// .y = lo | hi << 8. items[row][0].x holds the item count.
__device__ __forceinline__ int2 make_item(int phys_row, int lo, int hi) { return make_int2(phys_row, lo | (hi << 8)); }

struct SelArgs {
  const float* iq; const float* block_keys; const int* positions; const int* page_table;
  int* ids; int* n_sel; int2* items; float* scores_out;
  int batch, seq, idx_heads, ratio, topk, max_blocks, page_size, max_pages, max_items;
};

struct SelShared {
  float q[4 * IDX_D];
  float newkey[IDX_D];
  unsigned long long key[SEL_MAX_BLOCKS];
  int pages[SEL_MAX_BLOCKS];
  int sel[SEL_MAX_BLOCKS / 2];
};

// Selection for one query row at position p, by a whole SEL_NT-thread block.
// The indexer query must already be in S.q (heads past idx_heads zero). Block
// keys come from the cache, except block new_j (>= 0 when this very launch
// completed it), whose key is in S.newkey.
__device__ void select_row(const SelArgs& A, SelShared& S, int row, int b, int p, int new_j) {
  const int tid = threadIdx.x;
  const int n_elig = min((p + 1) / A.ratio, A.max_blocks);
  const int n_sel = min(n_elig, A.topk);
  int* out_ids = A.ids + (long)row * A.topk;

  // the page-table row, needed to describe the attention items, comes in with the keys
  const int n_lpages = min(A.max_pages, (p + A.page_size) / A.page_size);
  if (A.items)
    for (int i = tid; i < n_lpages; i += SEL_NT) S.pages[i] = A.page_table[(long)b * A.max_pages + i];
  if (A.scores_out)
    for (int j = tid; j < A.max_blocks; j += SEL_NT)
      if (j >= n_elig) A.scores_out[(long)row * A.max_blocks + j] = -INFINITY;

  if (n_elig > A.topk || A.scores_out) {
    // 16 lanes per block, 8 channels each; a chunk of 128 blocks is loaded
    // before any of it is used so the loads overlap
    const int sub = tid & 15, grp = tid >> 4;
    const float* bk = A.block_keys + (long)b * A.max_blocks * IDX_D;
    for (int c0 = 0; c0 < n_elig; c0 += SEL_CHUNK) {
      float4 kb[8][2];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int j = c0 + grp + 16 * i;
        const float4* kr = reinterpret_cast<const float4*>(
            j == new_j ? S.newkey + sub * 8 : bk + (long)(j < n_elig ? j : 0) * IDX_D + sub * 8);
        if (j < n_elig) {
          kb[i][0] = kr[0];
          kb[i][1] = kr[1];
        } else {
          kb[i][0] = kb[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      __syncthreads();    // S.q and S.newkey visible
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int j = c0 + grp + 16 * i;
        const float kv[8] = {kb[i][0].x, kb[i][0].y, kb[i][0].z, kb[i][0].w,
                             kb[i][1].x, kb[i][1].y, kb[i][1].z, kb[i][1].w};
        float dots[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float* qh = S.q + h * IDX_D + sub * 8;
          float acc = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = fmaf(qh[e], kv[e], acc);
          dots[h] = row16_sum(acc);
        }
        if (sub == 0 && j < n_elig) {
          float sc = 0.f;
#pragma unroll
          for (int h = 0; h < 4; ++h)
            if (h < A.idx_heads) sc = add_rn(sc, fmaxf(dots[h], 0.f));
          sc = div_rn(sc, 11.313708498984761f);     // sqrt(128)
          if (A.scores_out) A.scores_out[(long)row * A.max_blocks + j] = sc;
          S.key[j] = sel_key(sc, j);
        }
      }
    }
  }
  __syncthreads();
  if (n_elig <= A.topk) {
    for (int i = tid; i < n_elig; i += SEL_NT) { out_ids[i] = i; S.sel[i] = i; }
  } else {
    // rank by counting: keys are distinct, rank = number of larger keys
    // (keys past n_elig are padded with 0, which no real key is below)
    for (int j = n_elig + tid; j < ((n_elig + 15) & ~15); j += SEL_NT) S.key[j] = 0ull;
    __syncthreads();
    for (int j = tid; j < n_elig; j += SEL_NT) {
      const unsigned long long kj = S.key[j];
      int rank = 0;
      for (int i = 0; i < n_elig; i += 16) {
        unsigned long long k16[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) k16[u] = S.key[i + u];
#pragma unroll
        for (int u = 0; u < 16; ++u) rank += k16[u] > kj ? 1 : 0;
      }
      if (rank < A.topk) { out_ids[rank] = j; S.sel[rank] = j; }
    }
  }
  if (tid == 0) A.n_sel[row] = n_sel;
  if (!A.items) return;
  __syncthreads();
  // attention items: the groups of every selected block in rank order, then the tail's
  int2* items = A.items + (long)row * A.max_items;
  const int gpb = A.ratio >= 32 ? A.ratio / 32 : 1;
  const int n_blk_items = n_sel * gpb;
  const int ts = ((p + 1) / A.ratio) * A.ratio;
  const int n_tail = ts > p ? 0 : (p >> 5) - (ts >> 5) + 1;
  const int n_items = n_blk_items + n_tail;
  for (int it = tid; it < n_items; it += SEL_NT) {
    int t0, lo, hi;
    if (it < n_blk_items) {
      const int bs = S.sel[it / gpb] * A.ratio;
      if (A.ratio >= 32) { t0 = bs + (it % gpb) * 32; lo = 0; hi = 32; }
      else { t0 = bs & ~31; lo = bs - t0; hi = lo + A.ratio; }
    } else {
      t0 = (ts & ~31) + (it - n_blk_items) * 32;
      lo = max(ts - t0, 0);
      hi = min(p + 1 - t0, 32);
    }
    const int page = S.pages[t0 / A.page_size];
    items[1 + it] = make_item(page * A.page_size + t0 % A.page_size, lo, hi);
  }
  if (tid == 0) items[0] = make_int2(n_items, 0);
}

__global__ __launch_bounds__(SEL_NT) void qsa_select_kernel(SelArgs A) {
  const int row = blockIdx.x;
  const int b = row / A.seq, s = row % A.seq;
  const int p = A.positions[b] + s;
  __shared__ SelShared S;
  for (int i = threadIdx.x; i < 4 * IDX_D; i += SEL_NT)
    S.q[i] = i < A.idx_heads * IDX_D ? A.iq[(long)row * A.idx_heads * IDX_D + i] : 0.f;
  __syncthreads();
  select_row(A, S, row, b, p, -1);
}

// Decode (one token per sequence) front end in one launch: the query, key and
// value heads of qsa_prep, plus one selector block per sequence that appends
// the raw indexer key, norms and ropes the indexer query, pools the block this
// token completes (if any) and runs the selection, all without a round trip
// through memory between them.
template <typename T>
__global__ __launch_bounds__(SEL_NT) void qsa_front_kernel(PrepArgs<T> A, SelArgs SA) {
  const int b = blockIdx.x;
  const int role = blockIdx.y;
  if (role < A.hq + A.hkv) {
    prep_head<T>(A, b, 0, role);
    return;
  }
  const int tid = threadIdx.x;
  const int p = A.positions[b];
  __shared__ SelShared S;
  __shared__ float s_x[QSA_D], s_y[QSA_D], s_scr[32];
  if (tid < IDX_D) A.raw_keys[((long)b * A.max_ctx + p) * IDX_D + tid] = A.ik[(long)b * IDX_D + tid];
  const float* cs = A.cos + (long)p * A.rope;
  const float* sn = A.sin + (long)p * A.rope;
  for (int h = 0; h < 4; ++h) {
    __syncthreads();
    if (h >= A.idx_heads) {
      if (tid < IDX_D) S.q[h * IDX_D + tid] = 0.f;
      continue;
    }
    if (tid < IDX_D) s_x[tid] = Act<T>::load(A.iq, ((long)b * A.idx_heads + h) * IDX_D + tid);
    const float y = norm_rope_row<T>(s_x, s_y, s_scr, IDX_D, A.iq_norm, A.eps, A.rope, cs, sn);
    if (tid < IDX_D) {
      S.q[h * IDX_D + tid] = y;
      A.iq_out[((long)b * A.idx_heads + h) * IDX_D + tid] = y;
    }
  }
  int new_j = -1;
  if ((p + 1) % A.ratio == 0) {
    new_j = p / A.ratio;
    __syncthreads();
    const float y = pool_block<T>(new_j, A.ratio, A.rope, A.eps, A.ik_norm, A.cos, A.sin,
                                  A.raw_keys + (long)b * A.max_ctx * IDX_D, A.ik + (long)b * IDX_D, p,
                                  A.block_keys + (long)b * A.max_blocks * IDX_D, s_x, s_y, s_scr);
    if (tid < IDX_D) S.newkey[tid] = y;
  }
  __syncthreads();
  select_row(SA, S, b, b, p, new_j);
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
constexpr int GQA = 8;          // query heads per kv head this kernel handles
constexpr int ATT_WAVES = 2;    // waves (one 32-token item each) per workgroup

struct AttnArgs {
  const uint16_t* q; const uint16_t* k_pool; const uint16_t* v_pool;
  const int2* items;
  float* part_o; float* part_ml;
  int batch, seq, hq, hkv, page_size, max_items, splits;
  float scale;
};

__device__ __forceinline__ bf16x8_t load_bf16x8(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}

// split s of (row, kv head g) handles items [s*W, s*W + W), one per wave; the
// waves merge their (max, sum, output) in LDS and write one partial
__global__ __launch_bounds__(64 * ATT_WAVES) void qsa_attend_kernel(AttnArgs A) {
  const int split = blockIdx.x, g = blockIdx.y, row = blockIdx.z;   // row = b * seq + s
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int col = lane & 15;        // query head within the group (8..15 are padding)
  const int quad = lane >> 4;       // which 8-wide k slice / 4-row output slice
  const int2* items = A.items + (long)row * A.max_items;
  const int item = split * ATT_WAVES + wv;

  __shared__ float s_m[ATT_WAVES][GQA], s_l[ATT_WAVES][GQA];
  __shared__ float s_acc[ATT_WAVES][GQA][QSA_D];

  // the item descriptor and the query are independent loads
  const int n_items = items[0].x;
  const int2 desc = items[1 + min(item, A.max_items - 2)];
  bf16x8_t qhi[8], qlo[8];
  {
    const int hq = g * GQA + (col < GQA ? col : 0);
    const uint16_t* qh = A.q + ((long)(2 * row) * A.hq + hq) * QSA_D + 8 * quad;
    const uint16_t* ql = A.q + ((long)(2 * row + 1) * A.hq + hq) * QSA_D + 8 * quad;
    const bf16x8_t zero = {};
#pragma unroll
    for (int sk = 0; sk < 8; ++sk) {
      qhi[sk] = col < GQA ? load_bf16x8(qh + 32 * sk) : zero;
      qlo[sk] = col < GQA ? load_bf16x8(ql + 32 * sk) : zero;
    }
  }

  f32x4_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  if (item < n_items) {
    const int page = desc.x / A.page_size, row0 = desc.x % A.page_size;
    const int lo = desc.y & 0xff, hi = desc.y >> 8;
    const uint16_t* kp = A.k_pool + (((long)page * A.hkv + g) * A.page_size + row0) * QSA_D;
    const uint16_t* vp = A.v_pool + ((long)page * A.hkv + g) * QSA_D * A.page_size + row0;
    bf16x8_t kf[2][8], vf[16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int sk = 0; sk < 8; ++sk) kf[t][sk] = load_bf16x8(kp + (16 * t + col) * QSA_D + 32 * sk + 8 * quad);
#pragma unroll
    for (int db = 0; db < 16; ++db) vf[db] = load_bf16x8(vp + (long)(16 * db + col) * A.page_size + 8 * quad);

    // scores: rows = tokens 16t + 4 quad + v, column = head col
    f32x4_t sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sk = 0; sk < 8; ++sk) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][sk], qhi[sk], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][sk], qlo[sk], c, 0, 0, 0);
      }
      sc[t] = c;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int tok = 16 * t + 4 * quad + v;
        const float x = (tok >= lo && tok < hi) ? sc[t][v] * A.scale : -INFINITY;
        sc[t][v] = x;
        mx = fmaxf(mx, x);
      }
    mx = xor32_max(xor16_max(mx));
    m_run = mx;
    bf16x8_t pf;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float pv = __expf(sc[t][v] - m_run);
        l_run += pv;
        pf[4 * t + v] = __builtin_bit_cast(__bf16, f32_to_bf16(pv));
      }
    // O^T[d][head] += V^T[d][tok] P^T[tok][head]
#pragma unroll
    for (int db = 0; db < 16; ++db) acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[db], pf, acc[db], 0, 0, 0);
  }
  l_run = xor32_sum(xor16_sum(l_run));

  // merge the workgroup's waves
  if (quad == 0 && col < GQA) { s_m[wv][col] = m_run; s_l[wv][col] = l_run; }
  __syncthreads();
  float M = -INFINITY;
  if (col < GQA) {
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, s_m[w][col]);
  }
  const float wself = (col < GQA && m_run != -INFINITY) ? __expf(m_run - M) : 0.f;
  if (col < GQA) {
#pragma unroll
    for (int db = 0; db < 16; ++db)
#pragma unroll
      for (int v = 0; v < 4; ++v) s_acc[wv][col][16 * db + 4 * quad + v] = acc[db][v] * wself;
  }
  __syncthreads();
  const long pbase = (((long)row * A.hkv + g) * A.splits + split) * GQA;
  for (int i = threadIdx.x; i < GQA * QSA_D; i += 64 * ATT_WAVES) {
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) o += s_acc[w][i / QSA_D][i % QSA_D];
    A.part_o[pbase * QSA_D + i] = o;
  }
  if (threadIdx.x < GQA) {
    const int hh = threadIdx.x;
    float Mh = -INFINITY, L = 0.f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) Mh = fmaxf(Mh, s_m[w][hh]);
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w)
      if (s_m[w][hh] != -INFINITY) L += s_l[w][hh] * __expf(s_m[w][hh] - Mh);
    A.part_ml[(pbase + hh) * 2 + 0] = Mh;
    A.part_ml[(pbase + hh) * 2 + 1] = L;
  }
}

template <typename T>
struct CombineArgs {
  const float* part_o; const float* part_ml; const T* qg; T* out;
  int hq, hkv, splits;
};

constexpr int MAX_SPLITS = 1024;

template <typename T>
__global__ __launch_bounds__(QSA_D) void qsa_combine_kernel(CombineArgs<T> A) {
  const int hq = blockIdx.x, row = blockIdx.y;
  const int d = threadIdx.x;
  const int g = hq / GQA, hh = hq % GQA;
  const long base = (((long)row * A.hkv + g) * A.splits) * GQA + hh;
  __shared__ float s_w[MAX_SPLITS];
  __shared__ float s_red[QSA_D / 64];
  const float gate = Act<T>::load(A.qg, ((long)row * A.hq + hq) * (2 * QSA_D) + QSA_D + d);
  // every split's (max, sum) in parallel, then the weights in LDS
  float m = -INFINITY, l = 0.f;
  for (int s = d; s < A.splits; s += QSA_D) {
    const float ms = A.part_ml[(base + (long)s * GQA) * 2];
    m = fmaxf(m, ms);
    s_w[s] = ms;
  }
  m = wave_max(m);
  if ((d & 63) == 0) s_red[d >> 6] = m;
  __syncthreads();
  float M = s_red[0];
#pragma unroll
  for (int i = 1; i < QSA_D / 64; ++i) M = fmaxf(M, s_red[i]);
  for (int s = d; s < A.splits; s += QSA_D) {
    const float ms = s_w[s];
    const float w = ms == -INFINITY ? 0.f : __expf(ms - M);
    l += A.part_ml[(base + (long)s * GQA) * 2 + 1] * w;
    s_w[s] = w;
  }
  l = wave_sum(l);
  __syncthreads();
  if ((d & 63) == 0) s_red[d >> 6] = l;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int i = 0; i < QSA_D / 64; ++i) L += s_red[i];
  float o = 0.f;
#pragma unroll 8
  for (int s = 0; s < A.splits; ++s) o += A.part_o[(base + (long)s * GQA) * QSA_D + d] * s_w[s];
  const float att = Act<T>::round(o / L);
  const float sg = Act<T>::round(sigmoid_f(gate));
  Act<T>::store(A.out, ((long)row * A.hq + hq) * QSA_D + d, att * sg);
}

// ---------------------------------------------------------------------------
// fused decode step: one launch per token
// ---------------------------------------------------------------------------
// Grid (split, kv head g, sequence b); each 256-thread workgroup:
//   0. issues every load that depends only on the position: the indexer query
//      and key, its 8 query heads, the token's key and value, the first chunk
//      of block keys and the page-table row;
//   1. norms and ropes the indexer query (and pools the block this token
//      completes, if any) -- the same torch-order arithmetic as qsa_prep;
//   2. scores the eligible blocks and ranks them (every workgroup redundantly:
//      ~65 KB of L2-resident reads, cheaper than a cross-workgroup hand-off);
//   3. attends its four 32-token items (one per wave) on bf16 MFMA; the item
//      holding the current token takes that token's key/value from registers,
//      and split 0 of each kv head appends them to the pages;
//   4. writes its (max, sum, output) partial; the last workgroup of the kv head
//      to finish (agent-scope counter) merges all partials, applies the
//      sigmoid gate and resets the counter.
constexpr int DEC_WAVES = 4;
constexpr int DEC_NT = 64 * DEC_WAVES;
constexpr int DEC_MAX_BLOCKS = 2048;
constexpr int DEC_MAX_PAGES = 2048;
constexpr int DEC_MAX_TOPK = 256;
constexpr int DEC_MAX_SPLITS = 80;

template <typename T>
struct DecArgs {
  PrepArgs<T> P;
  float* part_o; float* part_ml; unsigned* counters; T* out;
  int* ids; int* n_sel; int2* items; float* iq_out;   // optional inspection outputs
  int splits, topk, max_items;
};

struct DecShared {
  float iq[4 * IDX_D];
  float newkey[IDX_D];
  float x[GQA * QSA_D];
  float y[GQA * QSA_D];
  float part[GQA * 32];
  float rinv[GQA];
  float knew[QSA_D], vnew[QSA_D];
  uint16_t qh[GQA * QSA_D], ql[GQA * QSA_D];
  int pages[DEC_MAX_PAGES];
  int sel[DEC_MAX_TOPK];
  union {
    unsigned long long key[DEC_MAX_BLOCKS];
    float acc[DEC_WAVES][GQA][QSA_D];
    float w[DEC_MAX_SPLITS][GQA];
  } u;
  float m[DEC_WAVES][GQA], l[DEC_WAVES][GQA];
  int last;
};

// y[r][e] = round_T(x[r][e] * rsqrt(mean_e x[r]^2 + eps) * w[e]) for R rows of n
// (n % 32 == 0, R * 32 <= blockDim), with the row sums of squares reduced in
// the order torch's CPU kernel uses (see torch_row_sumsq); then the first
// `rope` channels of every row rotated with (cs, sn). Called by the whole block.
template <typename T>
__device__ void norm_rope_rows(DecShared& sh, float* out, int R, int n, const float* w, float eps, int rope,
                               const float* cs, const float* sn) {
  const int t = threadIdx.x;
  __syncthreads();
  if (t < R * 32) {
    const int r = t >> 5, a = t & 31;
    float acc = 0.f;
    for (int e = a; e < n; e += 32) acc = add_rn(acc, mul_rn(sh.x[r * n + e], sh.x[r * n + e]));
    sh.part[t] = acc;
  }
  __syncthreads();
  if (t < R) {
    const float* pp = sh.part + t * 32;
    float tot = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const float c = add_rn(add_rn(add_rn(pp[l], pp[8 + l]), pp[16 + l]), pp[24 + l]);
      tot = l == 0 ? c : add_rn(tot, c);
    }
    sh.rinv[t] = rsqrt_rn(add_rn(div_rn(tot, (float)n), eps));
  }
  __syncthreads();
  for (int i = t; i < R * n; i += blockDim.x) {
    const int r = i / n, e = i % n;
    sh.y[i] = Act<T>::round(mul_rn(mul_rn(sh.x[i], sh.rinv[r]), w[e]));
  }
  __syncthreads();
  const int half = rope / 2;
  for (int i = t; i < R * n; i += blockDim.x) {
    const int r = i / n, e = i % n;
    float v = sh.y[i];
    if (e < rope) {
      const float rot = e < half ? -sh.y[r * n + e + half] : sh.y[r * n + e - half];
      v = add_rn(mul_rn(v, cs[e]), mul_rn(rot, sn[e]));
    }
    out[i] = v;
  }
  __syncthreads();
}

template <typename T>
__global__ __launch_bounds__(DEC_NT) void qsa_decode_kernel(DecArgs<T> D) {
  const PrepArgs<T>& A = D.P;
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int col = lane & 15, quad = lane >> 4;
  __shared__ DecShared sh;

  const int p = A.positions[b];
  const int ratio = A.ratio;
  const int n_elig = min((p + 1) / ratio, A.max_blocks);
  const int topk = D.topk;
  const int n_sel = min(n_elig, topk);
  const int j_new = (p + 1) % ratio == 0 ? p / ratio : -1;
  const bool leader = split == 0 && g == 0;       // writes the per-sequence side outputs
  const bool scoring = n_elig > topk;

  // ---- 0. loads that depend only on p
  float iqv[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = tid + DEC_NT * k;
    iqv[k] = i < A.idx_heads * IDX_D ? Act<T>::load(A.iq, (long)b * A.idx_heads * IDX_D + i) : 0.f;
  }
  const float ikv = tid < IDX_D ? Act<T>::load(A.ik, (long)b * IDX_D + tid) : 0.f;
  float qx[GQA];
#pragma unroll
  for (int h = 0; h < GQA; ++h) qx[h] = Act<T>::load(A.qg, ((long)b * A.hq + g * GQA + h) * (2 * QSA_D) + tid);
  const float kx = Act<T>::load(A.k_new, ((long)b * A.hkv + g) * QSA_D + tid);
  const float vx = Act<T>::load(A.v_new, ((long)b * A.hkv + g) * QSA_D + tid);
  const float* cs = A.cos + (long)p * A.rope;
  const float* sn = A.sin + (long)p * A.rope;
  const int sub = tid & 15, grp = tid >> 4;
  const float* bk = A.block_keys + (long)b * A.max_blocks * IDX_D;
  float4 kb[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int j = grp + 16 * i;
    if (scoring && j < n_elig && j != j_new) {
      const float4* kr = reinterpret_cast<const float4*>(bk + (long)j * IDX_D + sub * 8);
      kb[i][0] = kr[0];
      kb[i][1] = kr[1];
    } else {
      kb[i][0] = kb[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const int n_lpages = min(A.max_pages, (p + A.page_size) / A.page_size);
  for (int i = tid; i < n_lpages; i += DEC_NT) sh.pages[i] = A.page_table[(long)b * A.max_pages + i];

  // ---- 1. indexer query (and the block this token completes)
#pragma unroll
  for (int k = 0; k < 2; ++k) sh.x[tid + DEC_NT * k] = iqv[k];
  norm_rope_rows<T>(sh, sh.iq, 4, IDX_D, A.iq_norm, A.eps, A.rope, cs, sn);
  if (leader) {
    if (D.iq_out)
      for (int i = tid; i < A.idx_heads * IDX_D; i += DEC_NT) D.iq_out[(long)b * A.idx_heads * IDX_D + i] = sh.iq[i];
    if (tid < IDX_D) A.raw_keys[((long)b * A.max_ctx + p) * IDX_D + tid] = A.ik[(long)b * IDX_D + tid];
  }
  if (A.idx_heads < 4)
    for (int i = A.idx_heads * IDX_D + tid; i < 4 * IDX_D; i += DEC_NT) sh.iq[i] = 0.f;
  if (j_new >= 0) {
    // mean of the block's raw keys (16-row chunks in order), then norm + rope at its start
    const int t0 = j_new * ratio;
    if (tid < IDX_D) {
      const T* raw = A.raw_keys + (long)b * A.max_ctx * IDX_D;
      float total = 0.f;
      for (int c0 = 0; c0 < ratio; c0 += 16) {
        float acc = 0.f;
        const int c1 = min(c0 + 16, ratio);
        for (int i = c0; i < c1; ++i) {
          const int tok = t0 + i;
          acc = add_rn(acc, tok == p ? ikv : Act<T>::load(raw, (long)tok * IDX_D + tid));
        }
        total = c0 == 0 ? acc : add_rn(total, acc);
      }
      sh.x[tid] = Act<T>::round(div_rn(total, (float)ratio));
    }
    norm_rope_rows<T>(sh, sh.newkey, 1, IDX_D, A.ik_norm, A.eps, A.rope, A.cos + (long)t0 * A.rope,
                      A.sin + (long)t0 * A.rope);
    if (leader && tid < IDX_D) A.block_keys[((long)b * A.max_blocks + j_new) * IDX_D + tid] = sh.newkey[tid];
  }

  // ---- 2. block scores and top-k (ties to the lower index)
  if (scoring) {
    for (int c0 = 0; c0 < n_elig; c0 += SEL_CHUNK) {
      if (c0 > 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int j = c0 + grp + 16 * i;
          if (j < n_elig && j != j_new) {
            const float4* kr = reinterpret_cast<const float4*>(bk + (long)j * IDX_D + sub * 8);
            kb[i][0] = kr[0];
            kb[i][1] = kr[1];
          } else {
            kb[i][0] = kb[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int j = c0 + grp + 16 * i;
        if (j == j_new) {
          kb[i][0] = *reinterpret_cast<const float4*>(sh.newkey + sub * 8);
          kb[i][1] = *reinterpret_cast<const float4*>(sh.newkey + sub * 8 + 4);
        }
        const float kv[8] = {kb[i][0].x, kb[i][0].y, kb[i][0].z, kb[i][0].w,
                             kb[i][1].x, kb[i][1].y, kb[i][1].z, kb[i][1].w};
        float dots[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float* qh = sh.iq + h * IDX_D + sub * 8;
          float acc = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = fmaf(qh[e], kv[e], acc);
          dots[h] = row16_sum(acc);
        }
        if (sub == 0 && j < n_elig) {
          float sc = 0.f;
#pragma unroll
          for (int h = 0; h < 4; ++h)
            if (h < A.idx_heads) sc = add_rn(sc, fmaxf(dots[h], 0.f));
          sh.u.key[j] = sel_key(div_rn(sc, 11.313708498984761f), j);
        }
      }
    }
    for (int j = n_elig + tid; j < ((n_elig + 15) & ~15); j += DEC_NT) sh.u.key[j] = 0ull;
    __syncthreads();
    for (int j = tid; j < n_elig; j += DEC_NT) {
      const unsigned long long kj = sh.u.key[j];
      int rank = 0;
      for (int i = 0; i < n_elig; i += 16) {
        unsigned long long k16[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) k16[u] = sh.u.key[i + u];
#pragma unroll
        for (int u = 0; u < 16; ++u) rank += k16[u] > kj ? 1 : 0;
      }
      if (rank < topk) sh.sel[rank] = j;
    }
  } else {
    for (int i = tid; i < n_elig; i += DEC_NT) sh.sel[i] = i;
  }

  // ---- the query heads, key and value of this token (normed, roped)
#pragma unroll
  for (int h = 0; h < GQA; ++h) sh.x[h * QSA_D + tid] = qx[h];
  norm_rope_rows<T>(sh, sh.x, GQA, QSA_D, A.q_norm, A.eps, A.rope, cs, sn);   // roped rows land in x
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    const float yv = sh.x[h * QSA_D + tid];
    const uint16_t hi = f32_to_bf16(yv);
    sh.qh[h * QSA_D + tid] = hi;
    sh.ql[h * QSA_D + tid] = f32_to_bf16(yv - bf16_to_f32(hi));
  }
  __syncthreads();
  sh.x[tid] = kx;
  norm_rope_rows<T>(sh, sh.knew, 1, QSA_D, A.k_norm, A.eps, A.rope, cs, sn);
  sh.vnew[tid] = vx;
  const int pg_cur = sh.pages[p / A.page_size];
  const int prow = p % A.page_size;
  if (split == 0) {     // the token's key and value into its page slot, for later steps
    A.k_pool[(((long)pg_cur * A.hkv + g) * A.page_size + prow) * QSA_D + tid] = f32_to_bf16(sh.knew[tid]);
    A.v_pool[(((long)pg_cur * A.hkv + g) * QSA_D + tid) * A.page_size + v_slot(prow)] = f32_to_bf16(vx);
  }
  __syncthreads();

  // ---- 3. attention over this workgroup's items, one 32-token group per wave
  const int gpb = ratio >= 32 ? ratio / 32 : 1;
  const int n_blk_items = n_sel * gpb;
  const int ts = ((p + 1) / ratio) * ratio;
  const int n_tail = ts > p ? 0 : (p >> 5) - (ts >> 5) + 1;
  const int n_items = n_blk_items + n_tail;
  if (leader && D.items) {
    int2* items = D.items + (long)b * D.max_items;
    for (int it = tid; it < n_items; it += DEC_NT) {
      int t0, lo, hi;
      if (it < n_blk_items) {
        const int bs = sh.sel[it / gpb] * ratio;
        if (ratio >= 32) { t0 = bs + (it % gpb) * 32; lo = 0; hi = 32; }
        else { t0 = bs & ~31; lo = bs - t0; hi = lo + ratio; }
      } else {
        t0 = (ts & ~31) + (it - n_blk_items) * 32; lo = max(ts - t0, 0); hi = min(p + 1 - t0, 32);
      }
      items[1 + it] = make_item(sh.pages[t0 / A.page_size] * A.page_size + t0 % A.page_size, lo, hi);
    }
    if (tid == 0) items[0] = make_int2(n_items, 0);
  }
  if (leader && D.ids) {
    for (int i = tid; i < n_sel; i += DEC_NT) D.ids[(long)b * topk + i] = sh.sel[i];
    if (tid == 0) D.n_sel[b] = n_sel;
  }

  const int item = split * DEC_WAVES + wv;
  f32x4_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  if (item < n_items) {
    int t0, lo, hi;
    if (item < n_blk_items) {
      const int bs = sh.sel[item / gpb] * ratio;
      if (ratio >= 32) { t0 = bs + (item % gpb) * 32; lo = 0; hi = 32; }
      else { t0 = bs & ~31; lo = bs - t0; hi = lo + ratio; }
    } else {
      t0 = (ts & ~31) + (item - n_blk_items) * 32; lo = max(ts - t0, 0); hi = min(p + 1 - t0, 32);
    }
    const int page = sh.pages[t0 / A.page_size], row0 = t0 % A.page_size;
    const uint16_t* kp = A.k_pool + (((long)page * A.hkv + g) * A.page_size + row0) * QSA_D;
    const uint16_t* vp = A.v_pool + ((long)page * A.hkv + g) * QSA_D * A.page_size + row0;
    bf16x8_t kf[2][8], vf[16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int sk = 0; sk < 8; ++sk) kf[t][sk] = load_bf16x8(kp + (16 * t + col) * QSA_D + 32 * sk + 8 * quad);
#pragma unroll
    for (int db = 0; db < 16; ++db) vf[db] = load_bf16x8(vp + (long)(16 * db + col) * A.page_size + 8 * quad);
    // the current token's row comes from this launch, not from the pages
    if (p >= t0 && p < t0 + 32) {
      const int r = p - t0;
      if (col == (r & 15)) {
#pragma unroll
        for (int sk = 0; sk < 8; ++sk)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const __bf16 kv = __builtin_bit_cast(__bf16, f32_to_bf16(sh.knew[32 * sk + 8 * quad + e]));
            if (r >> 4) kf[1][sk][e] = kv; else kf[0][sk][e] = kv;
          }
      }
      const int kappa = v_slot(r);
      if (quad == (kappa >> 3)) {
#pragma unroll
        for (int db = 0; db < 16; ++db) vf[db][kappa & 7] = __builtin_bit_cast(__bf16, f32_to_bf16(sh.vnew[16 * db + col]));
      }
    }
    bf16x8_t qhi[8], qlo[8];
    const bf16x8_t zero = {};
#pragma unroll
    for (int sk = 0; sk < 8; ++sk) {
      qhi[sk] = col < GQA ? *reinterpret_cast<const bf16x8_t*>(sh.qh + col * QSA_D + 32 * sk + 8 * quad) : zero;
      qlo[sk] = col < GQA ? *reinterpret_cast<const bf16x8_t*>(sh.ql + col * QSA_D + 32 * sk + 8 * quad) : zero;
    }
    f32x4_t sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sk = 0; sk < 8; ++sk) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][sk], qhi[sk], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][sk], qlo[sk], c, 0, 0, 0);
      }
      sc[t] = c;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int tok = 16 * t + 4 * quad + v;
        const float x = (tok >= lo && tok < hi) ? sc[t][v] * (1.0f / 16.0f) : -INFINITY;
        sc[t][v] = x;
        mx = fmaxf(mx, x);
      }
    mx = xor32_max(xor16_max(mx));
    m_run = mx;
    bf16x8_t pf;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float pv = __expf(sc[t][v] - m_run);
        l_run += pv;
        pf[4 * t + v] = __builtin_bit_cast(__bf16, f32_to_bf16(pv));
      }
#pragma unroll
    for (int db = 0; db < 16; ++db) acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[db], pf, acc[db], 0, 0, 0);
  }
  l_run = xor32_sum(xor16_sum(l_run));

  // ---- 4. merge the waves, publish the partial, last workgroup combines
  __syncthreads();        // sh.u.key no longer read: reuse it for the wave merge
  if (quad == 0 && col < GQA) { sh.m[wv][col] = m_run; sh.l[wv][col] = l_run; }
  __syncthreads();
  if (col < GQA) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) M = fmaxf(M, sh.m[w][col]);
    const float wself = m_run == -INFINITY ? 0.f : __expf(m_run - M);
#pragma unroll
    for (int db = 0; db < 16; ++db)
#pragma unroll
      for (int v = 0; v < 4; ++v) sh.u.acc[wv][col][16 * db + 4 * quad + v] = acc[db][v] * wself;
  }
  __syncthreads();
  const long gbase = ((long)b * A.hkv + g) * D.splits;
  const long pbase = (gbase + split) * GQA;
  for (int i = tid; i < GQA * QSA_D; i += DEC_NT) {
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) o += sh.u.acc[w][i / QSA_D][i % QSA_D];
    D.part_o[pbase * QSA_D + i] = o;
  }
  if (tid < GQA) {
    float Mh = -INFINITY, L = 0.f;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) Mh = fmaxf(Mh, sh.m[w][tid]);
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w)
      if (sh.m[w][tid] != -INFINITY) L += sh.l[w][tid] * __expf(sh.m[w][tid] - Mh);
    D.part_ml[(pbase + tid) * 2 + 0] = Mh;
    D.part_ml[(pbase + tid) * 2 + 1] = L;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(D.counters + (long)b * A.hkv + g, 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    sh.last = prev == (unsigned)(D.splits - 1);
  }
  __syncthreads();
  if (!sh.last) return;
  __threadfence();
  // combine: weights per (split, head) in LDS, then every (head, d) sums its splits
  if (tid < GQA) {
    float M = -INFINITY;
    for (int s = 0; s < D.splits; ++s) M = fmaxf(M, D.part_ml[((gbase + s) * GQA + tid) * 2]);
    float L = 0.f;
    for (int s = 0; s < D.splits; ++s) {
      const float ms = D.part_ml[((gbase + s) * GQA + tid) * 2];
      const float w = ms == -INFINITY ? 0.f : __expf(ms - M);
      L += D.part_ml[((gbase + s) * GQA + tid) * 2 + 1] * w;
      sh.u.w[s][tid] = w;
    }
    sh.rinv[tid] = 1.0f / L;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    float o = 0.f;
    for (int s = 0; s < D.splits; ++s) o += D.part_o[((gbase + s) * GQA + h) * QSA_D + tid] * sh.u.w[s][h];
    const int hq = g * GQA + h;
    const float att = Act<T>::round(o * sh.rinv[h]);
    const float gate = Act<T>::round(sigmoid_f(Act<T>::load(A.qg, ((long)b * A.hq + hq) * (2 * QSA_D) + QSA_D + tid)));
    Act<T>::store(D.out, ((long)b * A.hq + hq) * QSA_D + tid, att * gate);
  }
  if (tid == 0) __hip_atomic_store(D.counters + (long)b * A.hkv + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int check_geom(const qm_qsa_geom* g, const char* who) {
  if (!g) return qm_fail(QM_ERR_ARG, who);
  if (g->head_dim != QSA_D || g->idx_dim != IDX_D)
    return qm_fail(QM_ERR_UNSUPPORTED, "qsa: head_dim must be 256 and idx_dim 128");
  if (g->n_kv_heads <= 0 || g->n_heads != g->n_kv_heads * GQA)
    return qm_fail(QM_ERR_UNSUPPORTED, "qsa: need 8 query heads per kv head");
  if (g->rope_dim <= 0 || g->rope_dim > IDX_D || g->rope_dim % 2)
    return qm_fail(QM_ERR_ARG, "qsa: rope_dim must be even and <= 128");
  if (g->idx_heads <= 0 || g->idx_heads > 4) return qm_fail(QM_ERR_UNSUPPORTED, "qsa: idx_heads must be 1..4");
  if (g->ratio <= 0 || (g->ratio % 32 && 32 % g->ratio))
    return qm_fail(QM_ERR_UNSUPPORTED, "qsa: ratio must divide 32 or be a multiple of 32");
  if (g->page_size <= 0 || g->page_size % 32) return qm_fail(QM_ERR_UNSUPPORTED, "qsa: page_size must be a multiple of 32");
  if (g->budget < g->ratio || g->budget % g->ratio) return qm_fail(QM_ERR_ARG, "qsa: budget must be a multiple of ratio");
  if (g->batch <= 0 || g->max_pages <= 0 || g->max_ctx <= 0 || g->max_blocks <= 0)
    return qm_fail(QM_ERR_ARG, "qsa: bad batch or capacity");
  if (g->act_dtype != QM_ACT_F32 && g->act_dtype != QM_ACT_BF16)
    return qm_fail(QM_ERR_DTYPE, "qsa: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
  return QM_OK;
}

// int2 entries per query row of the item table: a header, every group of the
// top-k blocks, and the tail's groups
int item_stride(const qm_qsa_geom* g) {
  const int gpb = g->ratio >= 32 ? g->ratio / 32 : 1;
  return 1 + (g->budget / g->ratio) * gpb + (g->ratio + 31) / 32 + 1;
}

template <typename T>
PrepArgs<T> prep_args(const qm_qsa_geom* g, int seq, const void* qg, const void* k_new, const void* v_new,
                      const void* iq, const void* ik, const float* q_norm, const float* k_norm, const float* iq_norm,
                      const float* ik_norm, const float* cos, const float* sin, const int* positions,
                      const int* page_table, void* k_pool, void* v_pool, void* raw_keys, float* block_keys,
                      void* q_out, float* iq_out) {
  PrepArgs<T> A;
  A.qg = static_cast<const T*>(qg); A.k_new = static_cast<const T*>(k_new); A.v_new = static_cast<const T*>(v_new);
  A.iq = static_cast<const T*>(iq); A.ik = static_cast<const T*>(ik);
  A.q_norm = q_norm; A.k_norm = k_norm; A.iq_norm = iq_norm; A.ik_norm = ik_norm;
  A.cos = cos; A.sin = sin; A.positions = positions; A.page_table = page_table;
  A.k_pool = static_cast<uint16_t*>(k_pool); A.v_pool = static_cast<uint16_t*>(v_pool);
  A.raw_keys = static_cast<T*>(raw_keys); A.block_keys = block_keys; A.q_out = static_cast<uint16_t*>(q_out);
  A.iq_out = iq_out;
  A.batch = g->batch; A.seq = seq; A.hq = g->n_heads; A.hkv = g->n_kv_heads; A.rope = g->rope_dim;
  A.idx_heads = g->idx_heads; A.ratio = g->ratio; A.page_size = g->page_size; A.max_pages = g->max_pages;
  A.max_ctx = g->max_ctx; A.max_blocks = g->max_blocks; A.eps = g->eps;
  return A;
}

template <typename T>
int launch_prep(const qm_qsa_geom* g, int seq, const void* qg, const void* k_new, const void* v_new, const void* iq,
                const void* ik, const float* q_norm, const float* k_norm, const float* iq_norm, const float* ik_norm,
                const float* cos, const float* sin, const int* positions, const int* page_table, void* k_pool,
                void* v_pool, void* raw_keys, float* block_keys, void* q_out, float* iq_out, hipStream_t stream) {
  PrepArgs<T> A = prep_args<T>(g, seq, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos, sin,
                               positions, page_table, k_pool, v_pool, raw_keys, block_keys, q_out, iq_out);
  dim3 grid(g->batch * seq, g->n_heads + g->n_kv_heads + 2);
  hipLaunchKernelGGL(qsa_prep_kernel<T>, grid, dim3(PREP_NT), 0, stream, A);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

SelArgs sel_args(const qm_qsa_geom* g, int seq, const float* iq, const float* block_keys, const int* positions,
                 const int* page_table, int* ids, int* n_sel, void* items, float* scores_out) {
  SelArgs A;
  A.iq = iq; A.block_keys = block_keys; A.positions = positions; A.page_table = page_table;
  A.ids = ids; A.n_sel = n_sel; A.items = static_cast<int2*>(items); A.scores_out = scores_out;
  A.batch = g->batch; A.seq = seq; A.idx_heads = g->idx_heads; A.ratio = g->ratio;
  A.topk = g->budget / g->ratio; A.max_blocks = g->max_blocks; A.page_size = g->page_size;
  A.max_pages = g->max_pages; A.max_items = item_stride(g);
  return A;
}

size_t part_o_bytes(const qm_qsa_geom* g, int rows, int splits) {
  return qm_align256((size_t)rows * g->n_kv_heads * splits * GQA * QSA_D * sizeof(float));
}



}  // namespace

extern "C" int qm_v_slot(int row) { return v_slot(row); }

extern "C" int qm_qsa_prep(const qm_qsa_geom* g, int seq, const void* qg, const void* k_new, const void* v_new,
                           const void* iq, const void* ik, const float* q_norm, const float* k_norm,
                           const float* iq_norm, const float* ik_norm, const float* cos, const float* sin,
                           const int* positions, const int* page_table, void* k_pool, void* v_pool, void* raw_keys,
                           float* block_keys, void* q_out, float* iq_out, hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_prep: null geometry");
  if (rc) return rc;
  if (seq <= 0) return qm_fail(QM_ERR_ARG, "qm_qsa_prep: seq must be positive");
  if (!iq || !ik || !iq_norm || !ik_norm || !cos || !sin || !positions || !raw_keys || !block_keys || !iq_out)
    return qm_fail(QM_ERR_ARG, "qm_qsa_prep: null indexer pointer");
  if (qg && (!q_norm || !q_out)) return qm_fail(QM_ERR_ARG, "qm_qsa_prep: qg needs q_norm and q_out");
  if ((k_new != nullptr) != (v_new != nullptr) || (k_new && (!k_norm || !page_table || !k_pool || !v_pool)))
    return qm_fail(QM_ERR_ARG, "qm_qsa_prep: k_new/v_new need k_norm, page_table and both pools");
  if (g->act_dtype == QM_ACT_F32)
    return launch_prep<float>(g, seq, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos, sin, positions,
                              page_table, k_pool, v_pool, raw_keys, block_keys, q_out, iq_out, stream);
  return launch_prep<bf16_t>(g, seq, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos, sin, positions,
                             page_table, k_pool, v_pool, raw_keys, block_keys, q_out, iq_out, stream);
}

extern "C" int qm_qsa_items_stride(const qm_qsa_geom* g) {
  if (!g || g->ratio <= 0 || g->budget < g->ratio) return 0;
  return item_stride(g);
}

extern "C" int qm_qsa_select(const qm_qsa_geom* g, int seq, const float* iq, const float* block_keys,
                             const int* positions, const int* page_table, int* ids, int* n_sel, void* items,
                             float* scores_out, hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_select: null geometry");
  if (rc) return rc;
  if (seq <= 0) return qm_fail(QM_ERR_ARG, "qm_qsa_select: seq must be positive");
  if (!iq || !block_keys || !positions || !ids || !n_sel) return qm_fail(QM_ERR_ARG, "qm_qsa_select: null pointer");
  if (items && !page_table) return qm_fail(QM_ERR_ARG, "qm_qsa_select: items need the page table");
  if (g->max_blocks > SEL_MAX_BLOCKS || g->max_pages > SEL_MAX_BLOCKS || g->budget / g->ratio > SEL_MAX_BLOCKS / 2)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_select: more than 4096 blocks or pages");
  SelArgs A = sel_args(g, seq, iq, block_keys, positions, page_table, ids, n_sel, items, scores_out);
  hipLaunchKernelGGL(qsa_select_kernel, dim3(g->batch * seq), dim3(SEL_NT), 0, stream, A);
  QM_CHECK_LAUNCH();
  return QM_OK;
}


namespace {
int items_at(const qm_qsa_geom* g, int p) {
  const int gpb = g->ratio >= 32 ? g->ratio / 32 : 1;
  const int topk = g->budget / g->ratio;
  const int n_elig = (p + 1) / g->ratio;
  const int sel = n_elig < topk ? n_elig : topk;
  const int ts = ((p + 1) / g->ratio) * g->ratio;
  const int tail = ts > p ? 0 : (p >> 5) - (ts >> 5) + 1;
  return sel * gpb + tail;
}
}  // namespace

extern "C" int qm_qsa_attend_splits(const qm_qsa_geom* g, int first_position, int last_position) {
  if (!g || g->ratio <= 0 || g->budget < g->ratio || first_position < 0 || last_position < first_position) return 1;
  int items = 0;
  if (last_position - first_position > 4 * g->ratio) {
    items = item_stride(g) - 1;   // every row of a long range reaches the bound
  } else {
    for (int p = first_position; p <= last_position; ++p) {
      const int n = items_at(g, p);
      items = n > items ? n : items;
    }
  }
  const int splits = (items + ATT_WAVES - 1) / ATT_WAVES;
  return splits < 1 ? 1 : splits;
}

extern "C" size_t qm_qsa_attend_workspace(const qm_qsa_geom* g, int seq, int splits) {
  if (!g || splits <= 0 || seq <= 0) return 0;
  const int rows = g->batch * seq;
  return part_o_bytes(g, rows, splits) + qm_align256((size_t)rows * g->n_kv_heads * splits * GQA * 2 * sizeof(float));
}

extern "C" int qm_qsa_attend(const qm_qsa_geom* g, int seq, const void* q, const void* qg, const void* k_pool,
                             const void* v_pool, const void* items, void* out, int splits, void* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_attend: null geometry");
  if (rc) return rc;
  if (!q || !qg || !k_pool || !v_pool || !items || !out) return qm_fail(QM_ERR_ARG, "qm_qsa_attend: null pointer");
  if (splits <= 0 || splits > MAX_SPLITS) return qm_fail(QM_ERR_ARG, "qm_qsa_attend: bad split count");
  if (seq <= 0 || (long)g->batch * seq > 65535) return qm_fail(QM_ERR_ARG, "qm_qsa_attend: bad seq");
  if (!workspace || workspace_bytes < qm_qsa_attend_workspace(g, seq, splits))
    return qm_fail(QM_ERR_WORKSPACE, "qm_qsa_attend: workspace too small");
  AttnArgs A;
  A.q = static_cast<const uint16_t*>(q); A.k_pool = static_cast<const uint16_t*>(k_pool);
  A.v_pool = static_cast<const uint16_t*>(v_pool); A.items = static_cast<const int2*>(items);
  A.part_o = static_cast<float*>(workspace);
  A.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_o_bytes(g, g->batch * seq, splits));
  A.batch = g->batch; A.seq = seq; A.hq = g->n_heads; A.hkv = g->n_kv_heads; A.page_size = g->page_size;
  A.max_items = item_stride(g); A.splits = splits;
  A.scale = 1.0f / 16.0f;   // 1/sqrt(256), exact
  hipLaunchKernelGGL(qsa_attend_kernel, dim3(splits, g->n_kv_heads, g->batch * seq), dim3(64 * ATT_WAVES), 0, stream,
                     A);
  QM_CHECK_LAUNCH();
  if (g->act_dtype == QM_ACT_F32) {
    CombineArgs<float> C{A.part_o, A.part_ml, static_cast<const float*>(qg), static_cast<float*>(out), g->n_heads,
                         g->n_kv_heads, splits};
    hipLaunchKernelGGL(qsa_combine_kernel<float>, dim3(g->n_heads, g->batch * seq), dim3(QSA_D), 0, stream, C);
  } else {
    CombineArgs<bf16_t> C{A.part_o, A.part_ml, static_cast<const bf16_t*>(qg), static_cast<bf16_t*>(out), g->n_heads,
                          g->n_kv_heads, splits};
    hipLaunchKernelGGL(qsa_combine_kernel<bf16_t>, dim3(g->n_heads, g->batch * seq), dim3(QSA_D), 0, stream, C);
  }
  QM_CHECK_LAUNCH();
  return QM_OK;
}

extern "C" int qm_qsa_pool_blocks(const qm_qsa_geom* g, const void* raw_keys, const float* k_norm, const float* cos,
                                  const float* sin, int first_block, int n_blocks, float* block_keys,
                                  hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_pool_blocks: null geometry");
  if (rc) return rc;
  if (!raw_keys || !k_norm || !cos || !sin || !block_keys) return qm_fail(QM_ERR_ARG, "qm_qsa_pool_blocks: null pointer");
  if (n_blocks <= 0) return QM_OK;
  if (first_block < 0 || first_block + n_blocks > g->max_blocks || (long)(first_block + n_blocks) * g->ratio > g->max_ctx)
    return qm_fail(QM_ERR_ARG, "qm_qsa_pool_blocks: block range outside the caches");
  if (g->act_dtype == QM_ACT_F32) {
    PoolArgs<float> A{static_cast<const float*>(raw_keys), k_norm, cos, sin, block_keys, first_block, n_blocks,
                      g->ratio, g->rope_dim, g->max_ctx, g->max_blocks, g->eps};
    hipLaunchKernelGGL(qsa_pool_kernel<float>, dim3(n_blocks, g->batch), dim3(IDX_D), 0, stream, A);
  } else {
    PoolArgs<bf16_t> A{static_cast<const bf16_t*>(raw_keys), k_norm, cos, sin, block_keys, first_block, n_blocks,
                       g->ratio, g->rope_dim, g->max_ctx, g->max_blocks, g->eps};
    hipLaunchKernelGGL(qsa_pool_kernel<bf16_t>, dim3(n_blocks, g->batch), dim3(IDX_D), 0, stream, A);
  }
  QM_CHECK_LAUNCH();
  return QM_OK;
}

extern "C" int qm_qsa_decode_front(const qm_qsa_geom* g, const void* qg, const void* k_new, const void* v_new,
                                   const void* iq, const void* ik, const float* q_norm, const float* k_norm,
                                   const float* iq_norm, const float* ik_norm, const float* cos, const float* sin,
                                   const int* positions, const int* page_table, void* k_pool, void* v_pool,
                                   void* raw_keys, float* block_keys, void* q_out, float* iq_out, int* ids,
                                   int* n_sel, void* items, hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_decode_front: null geometry");
  if (rc) return rc;
  if (!qg || !k_new || !v_new || !iq || !ik || !q_norm || !k_norm || !iq_norm || !ik_norm || !cos || !sin ||
      !positions || !page_table || !k_pool || !v_pool || !raw_keys || !block_keys || !q_out || !iq_out || !ids ||
      !n_sel || !items)
    return qm_fail(QM_ERR_ARG, "qm_qsa_decode_front: null pointer");
  if (g->max_blocks > SEL_MAX_BLOCKS || g->max_pages > SEL_MAX_BLOCKS || g->budget / g->ratio > SEL_MAX_BLOCKS / 2)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_decode_front: more than 4096 blocks or pages");
  const SelArgs S = sel_args(g, 1, iq_out, block_keys, positions, page_table, ids, n_sel, items, nullptr);
  dim3 grid(g->batch, g->n_heads + g->n_kv_heads + 1);
  if (g->act_dtype == QM_ACT_F32) {
    PrepArgs<float> A = prep_args<float>(g, 1, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos, sin,
                                         positions, page_table, k_pool, v_pool, raw_keys, block_keys, q_out, iq_out);
    hipLaunchKernelGGL(qsa_front_kernel<float>, grid, dim3(SEL_NT), 0, stream, A, S);
  } else {
    PrepArgs<bf16_t> A = prep_args<bf16_t>(g, 1, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos,
                                           sin, positions, page_table, k_pool, v_pool, raw_keys, block_keys, q_out,
                                           iq_out);
    hipLaunchKernelGGL(qsa_front_kernel<bf16_t>, grid, dim3(SEL_NT), 0, stream, A, S);
  }
  QM_CHECK_LAUNCH();
  return QM_OK;
}

extern "C" int qm_qsa_decode_splits(const qm_qsa_geom* g, int max_position) {
  if (!g || g->ratio <= 0 || g->budget < g->ratio || max_position < 0) return 1;
  const int n = (items_at(g, max_position) + DEC_WAVES - 1) / DEC_WAVES;
  return n < 1 ? 1 : n;
}

extern "C" size_t qm_qsa_decode_workspace(const qm_qsa_geom* g, int splits) {
  if (!g || splits <= 0) return 0;
  return part_o_bytes(g, g->batch, splits) + qm_align256((size_t)g->batch * g->n_kv_heads * splits * GQA * 2 * 4) +
         qm_align256((size_t)g->batch * g->n_kv_heads * sizeof(unsigned));
}

extern "C" int qm_qsa_decode(const qm_qsa_geom* g, const void* qg, const void* k_new, const void* v_new, const void* iq,
                             const void* ik, const float* q_norm, const float* k_norm, const float* iq_norm,
                             const float* ik_norm, const float* cos, const float* sin, const int* positions,
                             const int* page_table, void* k_pool, void* v_pool, void* raw_keys, float* block_keys,
                             void* out, int splits, void* workspace, size_t workspace_bytes, int* ids, int* n_sel,
                             void* items, float* iq_out, hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_decode: null geometry");
  if (rc) return rc;
  if (!qg || !k_new || !v_new || !iq || !ik || !q_norm || !k_norm || !iq_norm || !ik_norm || !cos || !sin ||
      !positions || !page_table || !k_pool || !v_pool || !raw_keys || !block_keys || !out)
    return qm_fail(QM_ERR_ARG, "qm_qsa_decode: null pointer");
  if ((ids != nullptr) != (n_sel != nullptr)) return qm_fail(QM_ERR_ARG, "qm_qsa_decode: ids and n_sel go together");
  if (g->max_blocks > DEC_MAX_BLOCKS || g->max_pages > DEC_MAX_PAGES || g->budget / g->ratio > DEC_MAX_TOPK)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_decode: more than 2048 blocks or pages, or top-k above 256 "
                                       "(use qm_qsa_prep + qm_qsa_select + qm_qsa_attend)");
  if (splits <= 0 || splits > DEC_MAX_SPLITS) return qm_fail(QM_ERR_ARG, "qm_qsa_decode: bad split count");
  if (!workspace || workspace_bytes < qm_qsa_decode_workspace(g, splits))
    return qm_fail(QM_ERR_WORKSPACE, "qm_qsa_decode: workspace too small");
  // counters first, at an offset that does not depend on the split count
  char* ws = static_cast<char*>(workspace);
  const size_t c_bytes = qm_align256((size_t)g->batch * g->n_kv_heads * sizeof(unsigned));
  const size_t ml_bytes = qm_align256((size_t)g->batch * g->n_kv_heads * splits * GQA * 2 * 4);
  dim3 grid(splits, g->n_kv_heads, g->batch);
  auto fill = [&](auto& D) {
    D.counters = reinterpret_cast<unsigned*>(ws);
    D.part_ml = reinterpret_cast<float*>(ws + c_bytes);
    D.part_o = reinterpret_cast<float*>(ws + c_bytes + ml_bytes);
    D.ids = ids; D.n_sel = n_sel; D.items = static_cast<int2*>(items); D.iq_out = iq_out;
    D.splits = splits; D.topk = g->budget / g->ratio; D.max_items = item_stride(g);
  };
  if (g->act_dtype == QM_ACT_F32) {
    DecArgs<float> D;
    D.P = prep_args<float>(g, 1, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos, sin, positions,
                           page_table, k_pool, v_pool, raw_keys, block_keys, nullptr, nullptr);
    D.out = static_cast<float*>(out);
    fill(D);
    hipLaunchKernelGGL(qsa_decode_kernel<float>, grid, dim3(DEC_NT), 0, stream, D);
  } else {
    DecArgs<bf16_t> D;
    D.P = prep_args<bf16_t>(g, 1, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos, sin, positions,
                            page_table, k_pool, v_pool, raw_keys, block_keys, nullptr, nullptr);
    D.out = static_cast<bf16_t*>(out);
    fill(D);
    hipLaunchKernelGGL(qsa_decode_kernel<bf16_t>, grid, dim3(DEC_NT), 0, stream, D);
  }
  QM_CHECK_LAUNCH();
  return QM_OK;
}
