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
__device__ void pool_block(int j, int ratio, int rope, float eps, const float* k_norm, const float* cos,
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
}

template <typename T>
struct PrepArgs {
  const T* qg; const T* k_new; const T* v_new; const T* iq; const T* ik;
  const float* q_norm; const float* k_norm; const float* iq_norm; const float* ik_norm;
  const float* cos; const float* sin;
  const int* positions; const int* page_table;
  uint16_t* k_pool; uint16_t* v_pool; T* raw_keys; float* block_keys;
  float* q_out; float* iq_out;
  int batch, seq, hq, hkv, rope, idx_heads, ratio, page_size, max_pages, max_ctx, max_blocks;
  float eps;
};

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

  if (role < A.hq) {
    // -------- attention query head `role`
    if (!A.qg) return;
    const T* src = A.qg + ((long)row * A.hq + role) * (2 * QSA_D);
    s_x[tid] = Act<T>::load(src, tid);
    const float y = norm_rope_row<T>(s_x, s_y, s_scr, QSA_D, A.q_norm, A.eps, A.rope, cs, sn);
    A.q_out[((long)row * A.hq + role) * QSA_D + tid] = y;
    return;
  }
  if (role < A.hq + A.hkv) {
    // -------- key/value head g: norm + rope the key, append both to the pages
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

__device__ __forceinline__ unsigned long long sel_key(float s, int j) {
  unsigned u = __float_as_uint(s);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);     // order-preserving
  return (static_cast<unsigned long long>(u) << 32) | static_cast<unsigned>(0x7fffffff - j);
}

struct SelArgs {
  const float* iq; const float* block_keys; const int* positions;
  int* ids; int* n_sel; float* scores_out;
  int batch, seq, idx_heads, ratio, topk, max_blocks;
};

__global__ __launch_bounds__(SEL_NT) void qsa_select_kernel(SelArgs A) {
  const int row = blockIdx.x;
  const int b = row / A.seq, s = row % A.seq;
  const int p = A.positions[b] + s;
  const int tid = threadIdx.x;
  const int n_elig = min((p + 1) / A.ratio, A.max_blocks);
  int* out_ids = A.ids + (long)row * A.topk;

  __shared__ float s_q[4 * IDX_D];
  __shared__ unsigned long long s_key[SEL_MAX_BLOCKS];

  if (A.scores_out) {
    for (int j = tid; j < A.max_blocks; j += SEL_NT)
      if (j >= n_elig) A.scores_out[(long)row * A.max_blocks + j] = -INFINITY;
  }
  if (n_elig <= A.topk && !A.scores_out) {
    for (int i = tid; i < n_elig; i += SEL_NT) out_ids[i] = i;
    if (tid == 0) A.n_sel[row] = n_elig;
    return;
  }
  for (int i = tid; i < A.idx_heads * IDX_D; i += SEL_NT) s_q[i] = A.iq[(long)row * A.idx_heads * IDX_D + i];
  __syncthreads();

  // 16 lanes per block, 8 channels each
  const int sub = tid & 15, grp = tid >> 4;
  const float* bk = A.block_keys + (long)b * A.max_blocks * IDX_D;
  for (int j0 = 0; j0 < n_elig; j0 += SEL_NT / 16) {
    const int j = j0 + grp;
    float dots[4] = {0.f, 0.f, 0.f, 0.f};
    if (j < n_elig) {
      const float4* kr = reinterpret_cast<const float4*>(bk + (long)j * IDX_D + sub * 8);
      const float4 k0 = kr[0], k1 = kr[1];
      const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      for (int h = 0; h < A.idx_heads; ++h) {
        const float* qh = s_q + h * IDX_D + sub * 8;
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(qh[e], kv[e], acc);
        dots[h] = acc;
      }
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1)
#pragma unroll
      for (int h = 0; h < 4; ++h) dots[h] += __shfl_xor(dots[h], off, 64);
    if (sub == 0 && j < n_elig) {
      float sc = 0.f;
      for (int h = 0; h < A.idx_heads; ++h) sc = add_rn(sc, fmaxf(dots[h], 0.f));
      sc = div_rn(sc, 11.313708498984761f);     // sqrt(128)
      if (A.scores_out) A.scores_out[(long)row * A.max_blocks + j] = sc;
      s_key[j] = sel_key(sc, j);
    }
  }
  if (n_elig <= A.topk) {
    for (int i = tid; i < n_elig; i += SEL_NT) out_ids[i] = i;
    if (tid == 0) A.n_sel[row] = n_elig;
    return;
  }
  __syncthreads();
  // rank by counting: keys are distinct, rank = number of larger keys
  for (int j = tid; j < n_elig; j += SEL_NT) {
    const unsigned long long kj = s_key[j];
    int rank = 0;
    for (int i = 0; i < n_elig; ++i) rank += s_key[i] > kj ? 1 : 0;
    if (rank < A.topk) out_ids[rank] = j;
  }
  if (tid == 0) A.n_sel[row] = A.topk;
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
constexpr int GQA = 8;          // query heads per kv head this kernel handles

struct AttnArgs {
  const float* q; const uint16_t* k_pool; const uint16_t* v_pool;
  const int* page_table; const int* positions; const int* ids; const int* n_sel;
  float* part_o; float* part_ml;
  int batch, seq, hq, hkv, ratio, page_size, max_pages, topk, splits;
  float scale;
};

// logical 32-token groups a query attends: selected blocks (in rank order),
// then the groups of its tail block
__device__ __forceinline__ int groups_per_block(int ratio) { return ratio >= 32 ? ratio / 32 : 1; }

__device__ __forceinline__ void item_range(const AttnArgs& A, int row, int item, int nsel_b, int p, int* t0,
                                           int* lo, int* hi) {
  const int gpb = groups_per_block(A.ratio);
  const int n_blk_items = nsel_b * gpb;
  if (item < n_blk_items) {
    const int j = A.ids[(long)row * A.topk + item / gpb];
    if (j < 0 || (long)(j + 1) * A.ratio > (long)p + 1) {   // not an eligible block: skip, never address it
      *t0 = -1; *lo = *hi = 0;
      return;
    }
    const int bs = j * A.ratio;
    if (A.ratio >= 32) {
      *t0 = bs + (item % gpb) * 32; *lo = 0; *hi = 32;
    } else {
      *t0 = bs & ~31; *lo = bs - *t0; *hi = *lo + A.ratio;
    }
    return;
  }
  const int ts = ((p + 1) / A.ratio) * A.ratio;
  const int g0 = ts & ~31;
  *t0 = g0 + (item - n_blk_items) * 32;
  *lo = max(ts - *t0, 0);
  *hi = min(p + 1 - *t0, 32);
}

__device__ __forceinline__ int n_items_for(const AttnArgs& A, int nsel_b, int p) {
  const int ts = ((p + 1) / A.ratio) * A.ratio;
  const int tail = ts > p ? 0 : (p >> 5) - (ts >> 5) + 1;
  return nsel_b * groups_per_block(A.ratio) + tail;
}

__device__ __forceinline__ bf16x8_t load_bf16x8(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}

__global__ __launch_bounds__(64) void qsa_attend_kernel(AttnArgs A) {
  const int split = blockIdx.x, g = blockIdx.y, row = blockIdx.z;   // row = b * seq + s
  const int b = row / A.seq;
  const int lane = threadIdx.x;
  const int col = lane & 15;        // query head within the group (8..15 are padding)
  const int quad = lane >> 4;       // which 8-wide k slice / 4-row output slice
  const int p = A.positions[b] + row % A.seq;
  const int nsel_b = A.n_sel[row];
  const int n_items = n_items_for(A, nsel_b, p);
  const int per = (n_items + A.splits - 1) / A.splits;
  const int it0 = split * per, it1 = min(n_items, it0 + per);

  // query fragments (B operand of S^T = K Q^T): hi and lo bf16 parts of
  // q[head col][32 s + 8 quad .. +8]
  bf16x8_t qhi[8], qlo[8];
  {
    const float* qrow = A.q + ((long)row * A.hq + g * GQA + (col < GQA ? col : 0)) * QSA_D;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = col < GQA ? qrow[32 * s + 8 * quad + e] : 0.f;
        const uint16_t hb = f32_to_bf16(x);
        const float rem = x - bf16_to_f32(hb);
        qhi[s][e] = __builtin_bit_cast(__bf16, hb);
        qlo[s][e] = __builtin_bit_cast(__bf16, f32_to_bf16(rem));
      }
    }
  }

  f32x4_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int item = it0; item < it1; ++item) {
    int t0, lo, hi;
    item_range(A, row, item, nsel_b, p, &t0, &lo, &hi);
    if (t0 < 0) continue;
    const int page = A.page_table[(long)b * A.max_pages + t0 / A.page_size];
    const int row0 = t0 % A.page_size;
    const uint16_t* kp = A.k_pool + (((long)page * A.hkv + g) * A.page_size + row0) * QSA_D;
    const uint16_t* vp = A.v_pool + ((long)page * A.hkv + g) * QSA_D * A.page_size + row0;

    // issue every K and V load of the group up front
    bf16x8_t kf[2][8], vf[16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s = 0; s < 8; ++s) kf[t][s] = load_bf16x8(kp + (16 * t + col) * QSA_D + 32 * s + 8 * quad);
#pragma unroll
    for (int db = 0; db < 16; ++db) vf[db] = load_bf16x8(vp + (long)(16 * db + col) * A.page_size + 8 * quad);

    // scores: rows = tokens 16t + 4 quad + v, column = head col
    f32x4_t sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][s], qhi[s], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][s], qlo[s], c, 0, 0, 0);
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
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __expf(m_run - m_new);
    float psum = 0.f;
    bf16x8_t pf;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float pv = __expf(sc[t][v] - m_new);
        psum += pv;
        pf[4 * t + v] = __builtin_bit_cast(__bf16, f32_to_bf16(pv));
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // O^T[d][head] += V^T[d][tok] P^T[tok][head]
#pragma unroll
    for (int db = 0; db < 16; ++db) {
      acc[db] *= alpha;
      acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[db], pf, acc[db], 0, 0, 0);
    }
  }
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  const long pbase = (((long)row * A.hkv + g) * A.splits + split) * GQA;
  if (col < GQA) {
    float* po = A.part_o + (pbase + col) * QSA_D;
#pragma unroll
    for (int db = 0; db < 16; ++db)
      *reinterpret_cast<float4*>(po + 16 * db + 4 * quad) =
          make_float4(acc[db][0], acc[db][1], acc[db][2], acc[db][3]);
    if (quad == 0) {
      A.part_ml[(pbase + col) * 2 + 0] = m_run;
      A.part_ml[(pbase + col) * 2 + 1] = l_run;
    }
  }
}

template <typename T>
struct CombineArgs {
  const float* part_o; const float* part_ml; const T* qg; T* out;
  int hq, hkv, splits;
};

template <typename T>
__global__ __launch_bounds__(QSA_D) void qsa_combine_kernel(CombineArgs<T> A) {
  const int hq = blockIdx.x, b = blockIdx.y;
  const int d = threadIdx.x;
  const int g = hq / GQA, hh = hq % GQA;
  const long base = (((long)b * A.hkv + g) * A.splits) * GQA + hh;
  float M = -INFINITY;
  for (int s = 0; s < A.splits; ++s) M = fmaxf(M, A.part_ml[(base + (long)s * GQA) * 2]);
  float L = 0.f, o = 0.f;
  for (int s = 0; s < A.splits; ++s) {
    const long ps = base + (long)s * GQA;
    const float m = A.part_ml[ps * 2];
    const float w = m == -INFINITY ? 0.f : __expf(m - M);
    L += A.part_ml[ps * 2 + 1] * w;
    o += A.part_o[ps * QSA_D + d] * w;
  }
  const float att = Act<T>::round(o / L);
  const float gate = Act<T>::load(A.qg, ((long)b * A.hq + hq) * (2 * QSA_D) + QSA_D + d);
  const float sg = Act<T>::round(sigmoid_f(gate));
  Act<T>::store(A.out, ((long)b * A.hq + hq) * QSA_D + d, att * sg);
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

template <typename T>
int launch_prep(const qm_qsa_geom* g, int seq, const void* qg, const void* k_new, const void* v_new, const void* iq,
                const void* ik, const float* q_norm, const float* k_norm, const float* iq_norm, const float* ik_norm,
                const float* cos, const float* sin, const int* positions, const int* page_table, void* k_pool,
                void* v_pool, void* raw_keys, float* block_keys, float* q_out, float* iq_out, hipStream_t stream) {
  PrepArgs<T> A;
  A.qg = static_cast<const T*>(qg); A.k_new = static_cast<const T*>(k_new); A.v_new = static_cast<const T*>(v_new);
  A.iq = static_cast<const T*>(iq); A.ik = static_cast<const T*>(ik);
  A.q_norm = q_norm; A.k_norm = k_norm; A.iq_norm = iq_norm; A.ik_norm = ik_norm;
  A.cos = cos; A.sin = sin; A.positions = positions; A.page_table = page_table;
  A.k_pool = static_cast<uint16_t*>(k_pool); A.v_pool = static_cast<uint16_t*>(v_pool);
  A.raw_keys = static_cast<T*>(raw_keys); A.block_keys = block_keys; A.q_out = q_out; A.iq_out = iq_out;
  A.batch = g->batch; A.seq = seq; A.hq = g->n_heads; A.hkv = g->n_kv_heads; A.rope = g->rope_dim;
  A.idx_heads = g->idx_heads; A.ratio = g->ratio; A.page_size = g->page_size; A.max_pages = g->max_pages;
  A.max_ctx = g->max_ctx; A.max_blocks = g->max_blocks; A.eps = g->eps;
  dim3 grid(g->batch * seq, g->n_heads + g->n_kv_heads + 2);
  hipLaunchKernelGGL(qsa_prep_kernel<T>, grid, dim3(PREP_NT), 0, stream, A);
  QM_CHECK_LAUNCH();
  return QM_OK;
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
                           float* block_keys, float* q_out, float* iq_out, hipStream_t stream) {
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

extern "C" int qm_qsa_select(const qm_qsa_geom* g, int seq, const float* iq, const float* block_keys,
                             const int* positions, int* ids, int* n_sel, float* scores_out, hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_select: null geometry");
  if (rc) return rc;
  if (seq <= 0) return qm_fail(QM_ERR_ARG, "qm_qsa_select: seq must be positive");
  if (!iq || !block_keys || !positions || !ids || !n_sel) return qm_fail(QM_ERR_ARG, "qm_qsa_select: null pointer");
  if (g->max_blocks > SEL_MAX_BLOCKS) return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_select: more than 4096 blocks");
  SelArgs A;
  A.iq = iq; A.block_keys = block_keys; A.positions = positions; A.ids = ids; A.n_sel = n_sel;
  A.scores_out = scores_out; A.batch = g->batch; A.seq = seq; A.idx_heads = g->idx_heads; A.ratio = g->ratio;
  A.topk = g->budget / g->ratio; A.max_blocks = g->max_blocks;
  hipLaunchKernelGGL(qsa_select_kernel, dim3(g->batch * seq), dim3(SEL_NT), 0, stream, A);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

extern "C" int qm_qsa_attend_splits(const qm_qsa_geom* g, int max_position) {
  if (!g || g->ratio <= 0) return 1;
  const int gpb = g->ratio >= 32 ? g->ratio / 32 : 1;
  const int topk = g->budget / g->ratio;
  const int n_elig = (max_position + 1) / g->ratio;
  const int sel = n_elig < topk ? n_elig : topk;
  const int tail_groups = (g->ratio + 31) / 32 + 1;
  int items = sel * gpb + tail_groups;
  return items < 1 ? 1 : items;
}

extern "C" size_t qm_qsa_attend_workspace(const qm_qsa_geom* g, int seq, int splits) {
  if (!g || splits <= 0 || seq <= 0) return 0;
  const int rows = g->batch * seq;
  return part_o_bytes(g, rows, splits) + qm_align256((size_t)rows * g->n_kv_heads * splits * GQA * 2 * sizeof(float));
}

extern "C" int qm_qsa_attend(const qm_qsa_geom* g, int seq, const float* q, const void* qg, const void* k_pool,
                             const void* v_pool, const int* page_table, const int* positions, const int* ids,
                             const int* n_sel, void* out, int splits, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_attend: null geometry");
  if (rc) return rc;
  if (!q || !qg || !k_pool || !v_pool || !page_table || !positions || !ids || !n_sel || !out)
    return qm_fail(QM_ERR_ARG, "qm_qsa_attend: null pointer");
  if (splits <= 0 || splits > 65535) return qm_fail(QM_ERR_ARG, "qm_qsa_attend: bad split count");
  if (seq <= 0 || (long)g->batch * seq > 65535) return qm_fail(QM_ERR_ARG, "qm_qsa_attend: bad seq");
  if (!workspace || workspace_bytes < qm_qsa_attend_workspace(g, seq, splits))
    return qm_fail(QM_ERR_WORKSPACE, "qm_qsa_attend: workspace too small");
  AttnArgs A;
  A.q = q; A.k_pool = static_cast<const uint16_t*>(k_pool); A.v_pool = static_cast<const uint16_t*>(v_pool);
  A.page_table = page_table; A.positions = positions; A.ids = ids; A.n_sel = n_sel;
  A.part_o = static_cast<float*>(workspace);
  A.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_o_bytes(g, g->batch * seq, splits));
  A.batch = g->batch; A.seq = seq; A.hq = g->n_heads; A.hkv = g->n_kv_heads; A.ratio = g->ratio; A.page_size = g->page_size;
  A.max_pages = g->max_pages; A.topk = g->budget / g->ratio; A.splits = splits;
  A.scale = 1.0f / 16.0f;   // 1/sqrt(256), exact
  hipLaunchKernelGGL(qsa_attend_kernel, dim3(splits, g->n_kv_heads, g->batch * seq), dim3(64), 0, stream, A);
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
