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

#include <type_traits>

#include "common.h"
#include "qwen4mix_internal.h"

namespace {

// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

constexpr int QSA_D = 256;     // attention head dim
constexpr int GQA = 8;          // query heads per kv head the attention kernels handle
constexpr int IDX_D = 128;     // indexer head dim
constexpr int PREP_NT = 256;

// column of page row `row` in a transposed V page: tokens of each 32-row group
// are stored in the order the PV MFMA's k index visits them
__host__ __device__ __forceinline__ int v_slot(int row) {
  const int t = row & 31;
  return (row & ~31) + 8 * ((t & 15) >> 2) + 4 * (t >> 4) + (t & 3);
}

// Block-key rows (the pooled, normed, roped indexer key of each block, 128
// floats) are kept permuted: element d at (d % 16) * 8 + d / 16, so that the
// 16 lanes that score a block for one query row (lane m owns elements m,
// m + 16, ..., m + 112) each read 32 contiguous bytes.
__host__ __device__ __forceinline__ int bk_index(int d) { return (d & 15) * 8 + (d >> 4); }

// Page layouts (one page of one kv head = P x 256 bf16): both pools keep their
// MFMA operands in lane order, so every wave-wide 16-byte load reads 1 KB of
// contiguous memory.
//   K: 16-token tiles x 8 steps of 32 channels; (tile, step) holds the A
//      operand of one 16x16x32 MFMA, lane = token % 16 + 16 * channel octet.
//   V: 32-token groups x 16 blocks of 16 channels; (group, block) holds the A
//      operand of the PV MFMA, lane = channel % 16 + 16 * slot octet, the
//      tokens of a group in v_slot order.
__host__ __device__ __forceinline__ int k_page_index(int row, int dim) {
  return ((((row >> 4) * 8 + (dim >> 5)) * 64 + (row & 15) + 16 * ((dim & 31) >> 3)) << 3) + (dim & 7);
}
__host__ __device__ __forceinline__ int v_page_index(int row, int dim) {
  const int s = v_slot(row) & 31;
  return ((((row >> 5) * 16 + (dim >> 4)) * 64 + (dim & 15) + 16 * (s >> 3)) << 3) + (s & 7);
}

// The bf16 query (hi and lo) as the attention MFMA's B operand reads it: per
// (row, kv head g, hi/lo, 32-channel step sk) 512 contiguous bytes holding
// [channel octet][head of the group][8 channels], so one wave-wide 16-byte load
// of a row's 8 heads reads 512 contiguous bytes. 16 KB per row at Hkv = 2.
__host__ __device__ __forceinline__ long q_index(long row, int hkv, int h2, int hq, int d) {
  const int g = hq >> 3, hh = hq & 7, sk = d >> 5, oct = (d >> 3) & 3, e = d & 7;
  return ((((((row * hkv + g) * 2 + h2) * 8 + sk) * 4 + oct) * 8 + hh) << 3) + e;
}
constexpr int Q_SK_STRIDE = 4 * 8 * 8;   // elements between 32-channel steps

// y = rope(round_T(rms_norm(x) * w)) for one row of `n` channels held in LDS
// by threads 0..n-1 (n <= blockDim). Rotates the first `rope` channels; c and
// s are this thread's cos and sin (rope_cs), loaded by the caller with its
// first loads. Returns the value of channel tid (0 for tid >= n).
template <typename T>
__device__ float norm_rope_row(float* s_x, float* s_y, float* s_scr, int n, const float* w, float eps,
                               int rope, float c, float s) {
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
    y = add_rn(mul_rn(y, c), mul_rn(rot, s));
  }
  return y;
}

// ---- RMS norms of one row per wave, in torch's CPU order: 32 partial sums,
// partial a summing the squares of elements a, a + 32, a + 64, ... in order;
// then c_l = ((s_l + s_(l+8)) + s_(l+16)) + s_(l+24) for l < 8, added in
// order; every square and sum rounded on its own. A 128-wide row sits in the
// wave as x[k] = element lane + 64 k (k < 2), a 256-wide row k < 4.
template <int N>
__device__ __forceinline__ float row_shl(float v) { return dpp_f<0x100 + N>(v); }

__device__ __forceinline__ float xor32_f(float v) { return lane_xor32(v); }

__device__ __forceinline__ float wave_rinv_finish(float s, float n, float eps) {
  const float s16 = lane_xor16(s);    // lanes 0..7 read lanes 16..23
  const float c = add_rn(add_rn(add_rn(s, row_shl<8>(s)), s16), row_shl<8>(s16));   // lanes 0..7: c_l
  float tot = readlane_f(c, 0);
#pragma unroll
  for (int l = 1; l < 8; ++l) tot = add_rn(tot, readlane_f(c, l));
  return rsqrt_rn(add_rn(div_rn(tot, n), eps));
}

template <int K>
__device__ __forceinline__ float wave_rinv(const float (&x)[K], float eps) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float q = mul_rn(x[k], x[k]);
    s = k == 0 ? q : add_rn(s, q);          // element lane + 64 k
    s = add_rn(s, xor32_f(q));              // element lane + 64 k + 32
  }
  return wave_rinv_finish(s, 64.f * K, eps);
}

// 1/sqrt(mean(x^2) + eps) of a 256-wide row held as x[k] = element lane + 64 k,
// for the attention query heads, whose rounding the attention's tolerance
// absorbs: fused multiply-adds, a lane tree and the hardware reciprocal square
// root (the rows whose bits are kept, the indexer's and the appended key, use
// wave_rinv)
__device__ __forceinline__ float wave_rinv_fast(const float (&x)[4], float eps) {
  float s = x[0] * x[0];
  s = fmaf(x[1], x[1], s);
  s = fmaf(x[2], x[2], s);
  s = fmaf(x[3], x[3], s);
  s = xor32_sum(xor16_sum(row16_sum(s)));
  return __builtin_amdgcn_rsqf(s * (1.0f / 256.0f) + eps);
}

// rope of a normed row held as y[k] = element lane + 64 k: element e < rope
// becomes y_e cos + (e < rope/2 ? -y_p : y_p) sin, p = e +- rope/2 (the
// partner's normed value, from lane p % 64 of register p / 64); every multiply
// and add rounded on its own.
template <int K>
__device__ __forceinline__ void wave_rope(float (&y)[K], int rope, const float (&cs)[2], const float (&sn)[2]) {
  const int lane = threadIdx.x & 63, half = rope >> 1;
  if (rope == 64) {
    // partner of element lane < 64 is lane ^ 32 of the same register; elements
    // 64 and up are not rotated
    const float yp = lane_xor32(y[0]);
    y[0] = add_rn(mul_rn(y[0], cs[0]), mul_rn(lane < 32 ? -yp : yp, sn[0]));
    return;
  }
  if (rope == 128) {
    // partner of element lane + 64 k is element lane + 64 (1 - k): same lane
    const float y0 = y[0], y1 = y[1];
    y[0] = add_rn(mul_rn(y0, cs[0]), mul_rn(-y1, sn[0]));
    y[1] = add_rn(mul_rn(y1, cs[1]), mul_rn(y0, sn[1]));
    return;
  }
  float out[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int e = lane + 64 * k;
    const int pe = min(e < half ? e + half : e - half, 127);
    const float v0 = __shfl(y[0], pe & 63, 64);
    const float v1 = __shfl(y[1], pe & 63, 64);
    const float yp = pe >= 64 ? v1 : v0;
    out[k] = e < rope ? add_rn(mul_rn(y[k], cs[k]), mul_rn(e < half ? -yp : yp, sn[k])) : y[k];
  }
  y[0] = out[0];
  y[1] = out[1];
}

// this thread's cos and sin of a table row (channel clamped into the rope range)
__device__ __forceinline__ float2 rope_cs(const float* cos, const float* sin, long row, int rope) {
  const long i = row * rope + min((int)threadIdx.x, rope - 1);
  return make_float2(cos[i], sin[i]);
}

// The indexer key of block j (reference/model.py:289-294): the float32 mean
// of its `ratio` raw keys (16-row chunks summed in order, then the chunk sums in
// order, then divided by the count, as torch's CPU mean reduces them), cast to
// the key dtype, RMS-normed with k_norm, and roped at the block's first
// position. Rows at or after `new0` come from `fresh` (row t - new0), earlier
// ones from `cache`. Called by a whole block; threads 0..127 own a channel.
// Inlined into its callers: as a call its pointers would be generic, so every
// row would be a flat load with its address formed in between. `v`, when
// `use_pre`, holds the block's first 64 rows as loaded already (the prep
// kernel requests them before the position arrives); it is the rows' buffer
// either way.
template <typename T>
__device__ __forceinline__ float pool_block_rows(T (&v)[64], bool use_pre, bool store, int j, int ratio, int rope,
                                                 float eps, const float* k_norm, const float* cos, const float* sin,
                                                 const T* cache, const T* fresh, int new0, float* blocks, float* s_x,
                                                 float* s_y, float* s_scr) {
  const int tid = threadIdx.x;
  const int t0 = j * ratio;
  // (a workgroup that does not store may hold no block: its rope row is row 0)
  const float2 csv = rope_cs(cos, sin, store ? t0 : 0, rope);
  if (tid < IDX_D) {
    // 64 rows' loads are issued together: each row's source is chosen by
    // address, and rows past the block are clamped and not added
    float total = 0.f;
    for (int r0 = 0; r0 < ratio; r0 += 64) {
      // the rows as loaded (no conversion: a conversion next to its load
      // would wait for that load before the next is issued), into v unless
      // it holds them already
      if (!(use_pre && r0 == 0)) {
#pragma unroll
        for (int i = 0; i < 64; ++i) {
          const int tok = t0 + min(r0 + i, ratio - 1);
          const T* src = tok >= new0 ? fresh + (long)(tok - new0) * IDX_D : cache + (long)tok * IDX_D;
          v[i] = src[tid];
        }
      }
      // every row requested before the first sum (the scheduler would
      // otherwise start the chain early and wait for each row in turn)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int c0 = r0 + 16 * c;
        if (c0 < ratio) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) acc = c0 + i < ratio ? add_rn(acc, Act<T>::load(&v[16 * c + i], 0)) : acc;
          total = c0 == 0 ? acc : add_rn(total, acc);
        }
      }
    }
    s_x[tid] = Act<T>::round(div_rn(total, (float)ratio));
  }
  const float y = norm_rope_row<T>(s_x, s_y, s_scr, IDX_D, k_norm, eps, rope, csv.x, csv.y);
  if (store && tid < IDX_D) blocks[(long)j * IDX_D + bk_index(tid)] = y;
  return y;
}

template <typename T>
__device__ __forceinline__ float pool_block(int j, int ratio, int rope, float eps, const float* k_norm, const float* cos,
                                            const float* sin, const T* cache, const T* fresh, int new0, float* blocks,
                                            float* s_x, float* s_y, float* s_scr) {
  T v[64];
  return pool_block_rows<T>(v, false, true, j, ratio, rope, eps, k_norm, cos, sin, cache, fresh, new0, blocks, s_x,
                            s_y, s_scr);
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

// qsa_prep_kernel, a 1-D grid of 256-thread workgroups. The first
// batch * (seq / ratio + 1) pool the blocks the chunk's rows complete (the
// longest work, dispatched first): workgroup x takes the (x % per)-th block
// completed in sequence x / per, if there is one. Every later wave takes one
// (row, role): roles 0..Hq-1 the attention query heads (RMS norm, rope, bf16
// hi/lo), Hq..Hq+Hkv-1 a key/value head (norm + rope the key, append both to
// the pages), then the indexer query heads (the first of which also appends
// the row's raw indexer key). A wave normalises its row on its own (no
// barrier); the pooled key of a block does not read the raw keys this launch
// appends (rows of the chunk come from ik).
template <typename T>
__device__ void prep_wave(const PrepArgs<T>& A, int row, int role) {
  const int lane = threadIdx.x & 63;
  const int b = row / A.seq, s = row % A.seq;
  const int pos = A.positions[b] + s;
  const int rope = A.rope;
  float cs[2], sn[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const long i = (long)pos * rope + min(lane + 64 * k, rope - 1);
    cs[k] = A.cos[i];
    sn[k] = A.sin[i];
  }
  auto nrm = [&](float xv, float ri, float w) { return Act<T>::round(mul_rn(mul_rn(xv, ri), w)); };
  if (role < A.hq) {
    if (!A.qg) return;
    const T* src = A.qg + ((long)row * A.hq + role) * (2 * QSA_D);
    float x[4], w[4], y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[k] = Act<T>::load(src, lane + 64 * k);
      w[k] = A.q_norm[lane + 64 * k];
    }
    const float ri = wave_rinv<4>(x, A.eps);
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = nrm(x[k], ri, w[k]);
    wave_rope<4>(y, rope, cs, sn);
    // the attention MFMA takes q as bf16: kept as hi + lo, the product carries
    // ~16 mantissa bits
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int d = lane + 64 * k;
      const uint16_t hi = f32_to_bf16(y[k]);
      A.q_out[q_index(row, A.hkv, 0, role, d)] = hi;
      A.q_out[q_index(row, A.hkv, 1, role, d)] = f32_to_bf16(y[k] - bf16_to_f32(hi));
    }
    return;
  }
  if (role < A.hq + A.hkv) {
    if (!A.k_new) return;
    const int g = role - A.hq;
    const long src = ((long)row * A.hkv + g) * QSA_D;
    const int page = A.page_table[(long)b * A.max_pages + pos / A.page_size];
    float x[4], v[4], w[4], y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[k] = Act<T>::load(A.k_new, src + lane + 64 * k);
      v[k] = Act<T>::load(A.v_new, src + lane + 64 * k);
      w[k] = A.k_norm[lane + 64 * k];
    }
    const float ri = wave_rinv<4>(x, A.eps);
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = nrm(x[k], ri, w[k]);
    wave_rope<4>(y, rope, cs, sn);
    const int prow = pos % A.page_size;
    const long pbase = ((long)page * A.hkv + g) * A.page_size * QSA_D;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int d = lane + 64 * k;
      A.k_pool[pbase + k_page_index(prow, d)] = f32_to_bf16(y[k]);
      A.v_pool[pbase + v_page_index(prow, d)] = f32_to_bf16(v[k]);
    }
    return;
  }
  const int h = role - A.hq - A.hkv;
  const long src = ((long)row * A.idx_heads + h) * IDX_D;
  float x[2], w[2], y[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    x[k] = Act<T>::load(A.iq, src + lane + 64 * k);
    w[k] = A.iq_norm[lane + 64 * k];
  }
  if (h == 0) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
      A.raw_keys[((long)b * A.max_ctx + pos) * IDX_D + lane + 64 * k] = A.ik[(long)row * IDX_D + lane + 64 * k];
  }
  const float ri = wave_rinv<2>(x, A.eps);
#pragma unroll
  for (int k = 0; k < 2; ++k) y[k] = nrm(x[k], ri, w[k]);
  wave_rope<2>(y, rope, cs, sn);
#pragma unroll
  for (int k = 0; k < 2; ++k) A.iq_out[src + lane + 64 * k] = y[k];
}

__host__ __device__ __forceinline__ int prep_pool_per_seq(int seq, int ratio) { return seq / ratio + 1; }

template <typename T>
__global__ __launch_bounds__(PREP_NT) void qsa_prep_kernel(PrepArgs<T> A) {
  const int per = prep_pool_per_seq(A.seq, A.ratio);
  const int n_pool = A.batch * per;
  const int x = blockIdx.x;
  if (x < n_pool) {
    // the blocks j whose last row (j + 1) ratio - 1 lies in [pos0, pos0 + seq)
    __shared__ float s_x[IDX_D], s_y[IDX_D], s_scr[32];
    const int b = x / per, xr = x % per;
    const T* fresh = A.ik + (long)b * A.seq * IDX_D;
    const T* cache = A.raw_keys + (long)b * A.max_ctx * IDX_D;
    float* blocks = A.block_keys + (long)b * A.max_blocks * IDX_D;
    if (A.ratio > 64) {
      const int pos0 = A.positions[b];
      const int j = pos0 / A.ratio + xr;
      if ((j + 1) * A.ratio > pos0 + A.seq) return;
      pool_block<T>(j, A.ratio, A.rope, A.eps, A.ik_norm, A.cos, A.sin, cache, fresh, pos0, blocks, s_x, s_y, s_scr);
      return;
    }
    // When the chunk starts on a block boundary (prefill chunks do), block
    // pos0 / ratio + xr is chunk rows xr ratio .. xr ratio + ratio - 1: those
    // rows are requested before the position is known (one round trip
    // instead of two); otherwise the block is loaded once the position is in.
    // The position by a vector load issued first (a scalar load would be
    // waited for together with the kernel's argument loads, before the rows);
    // the rows by every thread (those past 128 repeat a column), so that no
    // load sits in a branch of its own.
    const int pos0 = __builtin_amdgcn_readfirstlane(
        (int)__builtin_amdgcn_raw_buffer_load_b32(dev_rsrc(A.positions + b, 4), 0, 0, 0));
    T pre[64];
    const int col = threadIdx.x & (IDX_D - 1);
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      const int r = min(xr * A.ratio + min(i, A.ratio - 1), A.seq - 1);
      pre[i] = fresh[(long)r * IDX_D + col];
    }
    const int j = pos0 / A.ratio + xr;
    // A workgroup past the chunk's completed blocks has nothing to store; it
    // still runs on its (in-bounds) requested rows rather than returning here,
    // which would let the compiler move those loads after the position's wait
    const bool has = (j + 1) * A.ratio <= pos0 + A.seq;
    pool_block_rows<T>(pre, !has || pos0 % A.ratio == 0, has, j, A.ratio, A.rope, A.eps, A.ik_norm, A.cos, A.sin,
                       cache, fresh, pos0, blocks, s_x, s_y, s_scr);
    return;
  }
  // (row, role) waves: 32-bit arithmetic, the host keeps their count below 2^31
  const unsigned roles = static_cast<unsigned>(A.hq + A.hkv + A.idx_heads);
  const unsigned wid = static_cast<unsigned>(x - n_pool) * (PREP_NT / 64) + (threadIdx.x >> 6);
  if (wid >= static_cast<unsigned>(A.batch * A.seq) * roles) return;
  prep_wave<T>(A, static_cast<int>(wid / roles), static_cast<int>(wid % roles));
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
constexpr int SEL_NT = 256;             // the decode front kernel (its prep roles need 256)
constexpr int SELP_NT = 1024;           // qsa_select_kernel: one row per workgroup
constexpr int SEL_MAX_BLOCKS = 4096;    // eligible blocks one query may score

__device__ __forceinline__ unsigned long long sel_key(float s, int j) {
  unsigned u = __float_as_uint(s);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);     // order-preserving
  return (static_cast<unsigned long long>(u) << 32) | static_cast<unsigned>(0x7fffffff - j);
}

// An attention work item: one 32-token group of one page, rows [lo, hi) visible.
// .x = physical pool row of the group's first token (page * P + row0),
// .y = lo | hi << 8. items[row][0].x holds the item count.
__device__ __forceinline__ int2 make_item(int phys_row, int lo, int hi) { return make_int2(phys_row, lo | (hi << 8)); }

// Block scores s_j = sum_h relu(q_h . k_j) / sqrt(128) in the summation orders
// of the reference's CPU path (torch's einsum, reference/model.py:297-298),
// which the golden score vectors pin bit for bit:
//  * one query row (a decode step): each dot product is 16 partial sums,
//    partial m accumulating elements m, m + 16, ..., m + 112 by fused
//    multiply-add in that order; partials m, m + 4, m + 8, m + 12 are added in
//    that order into c_(m mod 4); the dot product is (c0 + c1) + (c2 + c3);
//  * several query rows (a prefill chunk): one fused multiply-add chain over
//    elements 0 .. 127;
// then ((relu(D_0) + relu(D_1)) + relu(D_2)) + relu(D_3), divided by sqrt(128)
// rounded to float.
//
// One-row order: 16 lanes per block (a DPP row), lane m holding partial m: its
// key elements m + 16 i are 8 loads, and a row of lanes reads whole 64-byte
// runs. The lanes add the partials by row shifts (lane i reads lane i + n).
constexpr int SCORE_LANES = 16;                 // NT / 16 blocks per pass of NT threads
// passes of keys held in registers ahead of use: eight at 256 threads (the
// first 128 blocks); two at 1024, where a thread has 128 VGPRs
template <int NT> constexpr int score_pre() { return NT >= 1024 ? 2 : 8; }

// (an invalid j loads row 0, always allocated, and zeroes the result: the
// loads stay unconditional so later waits on them stay exact)
__device__ __forceinline__ void load_block_part(float (&k)[8], const float* bk, int j, bool valid) {
  const float4* src = reinterpret_cast<const float4*>(bk + (long)(valid ? j : 0) * IDX_D + 8 * (threadIdx.x & 15));
  const float4 a = src[0], c = src[1];
  const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) k[i] = valid ? v[i] : 0.f;
}


// the one-row score of the block whose 16 lanes call this (valid in lane 0 of
// the 16); q holds this lane's elements of the 4 query rows
__device__ __forceinline__ float row16_block_score(const float (&q)[4][8], const float (&k)[8], int idx_heads) {
  float p[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    p[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) p[h] = fmaf(q[h][i], k[i], p[h]);
  }
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    float c = add_rn(p[h], row_shl<4>(p[h]));
    c = add_rn(c, row_shl<8>(p[h]));
    c = add_rn(c, row_shl<12>(p[h]));           // lanes 0..3: c_0 .. c_3
    const float u = add_rn(c, row_shl<1>(c));     // lane 0: c0 + c1, lane 2: c2 + c3
    p[h] = add_rn(u, row_shl<2>(u));              // lane 0: the dot product
  }
  float sc = 0.f;
#pragma unroll
  for (int h = 0; h < 4; ++h)
    if (h < idx_heads) sc = add_rn(sc, fmaxf(p[h], 0.f));
  return div_rn(sc, 11.313708498984761f);     // sqrt(128) as a float
}

// keys[j] = sel_key(score_j, j) for every eligible block j (and scores_out[j]
// when given) in the one-row order, then zeros up to a multiple of 32. kp[u]
// comes in holding pass u's keys (load_block_part); later passes load PRE
// passes ahead of use. Block new_j's key is new_key (LDS), not the cache's.
// s_iq: 4 rows of 128.
template <int NT, int PRE>
__device__ void score_blocks(const float* s_iq, const float* new_key, const float* bk, int n_elig, int new_j,
                             int idx_heads, unsigned long long* keys, float* scores_out, float (&kp)[PRE][8]) {
  constexpr int SCORE_PASS = NT / SCORE_LANES;
  const int tid = threadIdx.x, jl = tid >> 4, m = tid & 15;
  float q[4][8];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) q[h][i] = s_iq[h * IDX_D + 16 * i + m];
  const int n_pass = (n_elig + SCORE_PASS - 1) / SCORE_PASS;
  for (int ps0 = 0; ps0 < n_pass; ps0 += PRE) {
#pragma unroll
    for (int u = 0; u < PRE; ++u) {
      const int ps = ps0 + u;
      if (ps < n_pass) {
        const int j = ps * SCORE_PASS + jl;
        if (j == new_j) {
#pragma unroll
          for (int i = 0; i < 8; ++i) kp[u][i] = new_key[16 * i + m];
        }
        const float sc = row16_block_score(q, kp[u], idx_heads);
        if (m == 0 && j < n_elig) {
          keys[j] = sel_key(sc, j);
          if (scores_out) scores_out[j] = sc;
        }
        const int jn = j + PRE * SCORE_PASS;
        if (ps + PRE < n_pass) load_block_part(kp[u], bk, jn, jn < n_elig && jn != new_j);
      }
    }
  }
  const int npad = (n_elig + 31) & ~31;
  for (int j = n_elig + tid; j < npad; j += NT) keys[j] = 0ull;
}

// The one-row dot products of the 4 query rows with the block of the calling
// 16 lanes (the order of row16_block_score), valid in lane 0 of the 16.
__device__ __forceinline__ float4 row16_dots(const float (&q)[4][8], const float (&k)[8]) {
  float p[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    p[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) p[h] = fmaf(q[h][i], k[i], p[h]);
  }
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    float c = add_rn(p[h], row_shl<4>(p[h]));
    c = add_rn(c, row_shl<8>(p[h]));
    c = add_rn(c, row_shl<12>(p[h]));
    const float u = add_rn(c, row_shl<1>(c));
    p[h] = add_rn(u, row_shl<2>(u));
  }
  return make_float4(p[0], p[1], p[2], p[3]);
}

// The top-k of at most 128 eligible blocks of one query row (ties to the lower
// index) from their dot products in dsc, by all 256 threads, written to
// sel[0 .. topk) in block order; returns the want-th selected block (block
// order; -1 for want < 0), the same in every thread. Ranking by counting:
// thread (wave w, lane l) takes block i = 32 w + (l & 31) and half h = l >> 5
// of the blocks. It forms block i's score key (relu, the heads added in order,
// the division by sqrt(128), then the order-preserving bits of sel_key; zero
// past n_elig, below every eligible key), the h = 0 lanes store the top 31
// bits of that key to LDS, and after a barrier each thread counts the keys of
// half h strictly above its own (four keys per broadcast LDS read; 31-bit
// keys, so a comparison is the sign bit of a difference). The halves' counts
// meet by a lane swap (l ^ 32). A block with fewer than topk keys above it is
// kept; each wave's kept blocks are one 32-bit ballot, published in masks
// (LDS, 4 words) behind a second barrier. The kept set holds every block
// above any kept one (its coarse key is at least as high, so fewer keys are
// above it), so when exactly topk blocks are kept it is the top-k and final.
// Otherwise blocks with equal coarse keys straddle the boundary, and every thread
// counts again with 64-bit keys (score bits over the reversed index, so that
// the lower index ranks higher), which orders every pair; a third barrier
// publishes those masks. A kept block's place in sel is the count of kept
// blocks below it; sel is published by the caller's next barrier.
__device__ __forceinline__ int select128(const float4* dsc, int n_elig, int idx_heads, int topk, int* sel,
                                         unsigned long long* keys, unsigned* masks, int want) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = 32 * wv + (lane & 31), h = lane >> 5;
  const float4 dd = dsc[i];
  const float dv[4] = {dd.x, dd.y, dd.z, dd.w};
  float sc = fmaxf(dv[0], 0.f);
#pragma unroll
  for (int hh = 1; hh < 4; ++hh) sc = hh < idx_heads ? add_rn(sc, fmaxf(dv[hh], 0.f)) : sc;
  const unsigned long long key = i < n_elig ? sel_key(div_rn(sc, 11.313708498984761f), i) : 0ull;
  // the score key's top 31 bits: a coarser order, which keeps the set exact
  // (below), and lets a comparison be a subtraction's sign bit
  const unsigned hk = static_cast<unsigned>(key >> 33);
  unsigned* hkeys = masks + 8;                       // 128 score keys after the mask words
  if (h == 0) { hkeys[i] = hk; keys[i] = key; }
  __syncthreads();
  QM_PHASE(3);
  // the 64 score keys of half h, all requested before the first compare;
  // (hk - k) >> 31 is 1 exactly when k > hk (both below 2^31), four
  // independent counts with no compare-and-carry chain through vcc
  {
    const uint4* kh = reinterpret_cast<const uint4*>(hkeys + 64 * h);
    uint4 kk[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) kk[q] = kh[q];
    __builtin_amdgcn_sched_barrier(0);
    unsigned c4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      c4[0] += (hk - kk[q].x) >> 31;
      c4[1] += (hk - kk[q].y) >> 31;
      c4[2] += (hk - kk[q].z) >> 31;
      c4[3] += (hk - kk[q].w) >> 31;
    }
    const unsigned cnt = (c4[0] + c4[1]) + (c4[2] + c4[3]);
    const auto sw = __builtin_amdgcn_permlane32_swap(cnt, cnt, false, false);
    const unsigned above = sw[0] + sw[1];
    const unsigned mine = static_cast<unsigned>(
        __builtin_amdgcn_ballot_w64(lane < 32 && i < n_elig && above < static_cast<unsigned>(topk)));
    if (lane == 0) masks[wv] = mine;
  }
  __syncthreads();
  unsigned m[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) m[w] = masks[w];
  if (__popc(m[0]) + __popc(m[1]) + __popc(m[2]) + __popc(m[3]) != static_cast<unsigned>(topk)) {
    // equal scores at the boundary: rank by the full keys
    const ulonglong2* kh = reinterpret_cast<const ulonglong2*>(keys + 64 * h);
    unsigned cnt = 0;
#pragma unroll 4
    for (int q = 0; q < 32; ++q) {
      const ulonglong2 kk = kh[q];
      cnt += (kk.x > key ? 1u : 0u) + (kk.y > key ? 1u : 0u);
    }
    const auto sw = __builtin_amdgcn_permlane32_swap(cnt, cnt, false, false);
    const unsigned rank = sw[0] + sw[1];
    const unsigned mine = static_cast<unsigned>(
        __builtin_amdgcn_ballot_w64(lane < 32 && i < n_elig && rank < static_cast<unsigned>(topk)));
    __syncthreads();                     // every thread has read the first masks
    if (lane == 0) masks[wv] = mine;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 4; ++w) m[w] = masks[w];
  }
  unsigned below = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) below += w < wv ? __popc(m[w]) : 0u;
  const unsigned mw = m[wv];
  if (lane < 32 && ((mw >> lane) & 1u)) sel[below + __builtin_amdgcn_mbcnt_lo(mw, 0u)] = i;
  if (want < 0) return -1;
  // the want-th kept block: its word, then its bit (the lane whose count of
  // kept bits below it is the remainder)
  int w = 0, n = want;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int c = __popc(m[w]);
    if (n >= c) { n -= c; ++w; }
  }
  const unsigned word = m[w];
  const unsigned long long hit = __builtin_amdgcn_ballot_w64(
      lane < 32 && ((word >> lane) & 1u) && __builtin_amdgcn_mbcnt_lo(word, 0u) == static_cast<unsigned>(n));
  return 32 * w + static_cast<int>(__builtin_ctzll(hit));
}

// keys[j] = sel_key(score_j, j) for every eligible block j in the one-row
// order, in rounds of PRE passes (PRE * NT / 16 blocks): the passes leave each
// block's 4 dot products in dsc (LDS), then one thread per block forms its
// score and key, so that the relu, sum and division run once per block rather
// than in all 16 of its lanes. kp[u] comes in holding pass u's keys; later
// rounds load one round ahead. Block new_j's key is new_key (LDS). Ends with
// the keys padded with zeros to a multiple of 32 (after a barrier the caller
// issues). Given sel, when one round of 128 holds every eligible block, the
// workgroup (NT = 256) selects the top-k from the round's dot products instead
// (select128) and the call returns true, with sel written (published by the
// caller's next barrier) and *blk = the want-th selected block in block order
// (want >= 0); keys[0 .. 128) and the 1 KB after them are then scratch.
template <int NT, int PRE>
__device__ bool score_block_rounds(const float* s_iq, const float* new_key, const float* bk, int n_elig, int new_j,
                                   int idx_heads, unsigned long long* keys, float4* dsc, float (&kp)[PRE][8],
                                   int topk = 0, int* sel = nullptr, int want = -1, int* blk = nullptr) {
  constexpr int PASS = NT / SCORE_LANES;
  constexpr int ROUND = PASS * PRE;
  const int tid = threadIdx.x, jl = tid >> 4, m = tid & 15;
  float q[4][8];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) q[h][i] = s_iq[h * IDX_D + 16 * i + m];
  for (int r0 = 0; r0 < n_elig; r0 += ROUND) {
    if (new_j >= r0 && new_j < r0 + ROUND) {
      // the block this launch completes is not in the cache yet: its key from LDS
#pragma unroll
      for (int u = 0; u < PRE; ++u)
        if (r0 + u * PASS + jl == new_j) {
#pragma unroll
          for (int i = 0; i < 8; ++i) kp[u][i] = new_key[16 * i + m];
        }
    }
    // every pass of the round at once (blocks past n_elig hold zeros), so that
    // their independent chains interleave
    float4 d[PRE];
#pragma unroll
    for (int u = 0; u < PRE; ++u) d[u] = row16_dots(q, kp[u]);
    QM_PHASE(11);
    if (m == 0) {
#pragma unroll
      for (int u = 0; u < PRE; ++u) dsc[u * PASS + jl] = d[u];
    }
    if (r0 + ROUND < n_elig) {
#pragma unroll
      for (int u = 0; u < PRE; ++u) {
        const int jn = r0 + ROUND + u * PASS + jl;
        load_block_part(kp[u], bk, jn, jn < n_elig && jn != new_j);
      }
    }
    QM_PHASE(13);
    __syncthreads();
    QM_PHASE(14);
    if constexpr (NT == 256 && ROUND == 128) {
      if (sel && n_elig <= ROUND) {
        *blk = select128(dsc, n_elig, idx_heads, topk, sel, keys, reinterpret_cast<unsigned*>(keys + ROUND), want);
        return true;
      }
    }
    for (int t = tid; t < ROUND && r0 + t < n_elig; t += NT) {
      const float4 dd = dsc[t];
      const float dv[4] = {dd.x, dd.y, dd.z, dd.w};
      float sc = 0.f;
#pragma unroll
      for (int h = 0; h < 4; ++h)
        if (h < idx_heads) sc = add_rn(sc, fmaxf(dv[h], 0.f));
      keys[r0 + t] = sel_key(div_rn(sc, 11.313708498984761f), r0 + t);
    }
    __syncthreads();
  }
  const int npad = (n_elig + 31) & ~31;
  for (int j = n_elig + tid; j < npad; j += NT) keys[j] = 0ull;
  return false;
}

// prefetch of the first PRE passes (issued before the scores are needed)
template <int NT, int PRE>
__device__ __forceinline__ void prefetch_block_keys(float (&kp)[PRE][8], const float* bk, int n_elig, int new_j,
                                                    bool on) {
  constexpr int SCORE_PASS = NT / SCORE_LANES;
  const int jl = threadIdx.x >> 4;
#pragma unroll
  for (int u = 0; u < PRE; ++u) {
    const int j = u * SCORE_PASS + jl;
    load_block_part(kp[u], bk, j, on && j < n_elig && j != new_j);
  }
}

// the decode kernel's prefetch of the first PRE passes: no zeroing (a block
// past the eligible ones is scored but never ranked, and the block this launch
// completes takes its key from LDS), rows past max_blocks, or every row when
// the launch never scores, read row 0
template <int NT, int PRE>
__device__ __forceinline__ void prefetch_block_keys_raw(float (&kp)[PRE][8], const float* bk, int max_blocks, bool on) {
  constexpr int SCORE_PASS = NT / SCORE_LANES;
  const int jl = threadIdx.x >> 4;
#pragma unroll
  for (int u = 0; u < PRE; ++u) {
    const int j = u * SCORE_PASS + jl;
    const float4* src =
        reinterpret_cast<const float4*>(bk + (long)(on && j < max_blocks ? j : 0) * IDX_D + 8 * (threadIdx.x & 15));
    const float4 a = src[0], c = src[1];
    kp[u][0] = a.x; kp[u][1] = a.y; kp[u][2] = a.z; kp[u][3] = a.w;
    kp[u][4] = c.x; kp[u][5] = c.y; kp[u][6] = c.z; kp[u][7] = c.w;
  }
}

// The several-rows order: one lane per (block, head) walks the block's 128
// elements in order in one fused multiply-add chain. Rounds of SEQ_RB blocks:
// the whole workgroup copies the round's block rows into LDS with coalesced
// loads (a lane walking its own 512-byte row in global memory would touch 64
// cache lines per load instruction), each row padded by 16 bytes so that the
// lanes' row reads fall on distinct banks; the next round's rows are loaded
// into registers while this round is scored. Waves 0..7 score: wave w takes
// head w % 4 and blocks 64 (w / 4) + lane, so the query row is the same in
// every lane and comes through the scalar cache (s_load) as a uniform operand
// of the multiply-adds. Each lane's relu'd dot product goes to
// dsc[head][block of the round], then one thread per block adds the heads in
// order, divides and forms the key.
constexpr int SEQ_RB = 128;                  // blocks per round
constexpr int SEQ_STRIDE = IDX_D + 4;        // floats per staged row
constexpr int SEQ_STAGE = SEQ_RB * SEQ_STRIDE;

template <int NT>
__device__ void score_blocks_seq(const float* __restrict__ iq_row, const float* bk, int n_elig, int idx_heads,
                                 unsigned long long* keys, float* scores_out, float (*dsc)[NT / 4],
                                 float* stage) {
  static_assert(NT == 1024 && NT / 4 >= SEQ_RB, "eight scoring waves of 64 blocks; dsc holds a round");
  constexpr int F4 = SEQ_RB * IDX_D / 4 / NT;  // float4 of a round each thread copies
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = wv & 3, sub = wv >> 2;
  // the row through the constant address space: a uniform address there is
  // read with scalar loads into SGPRs (the kernel never writes it)
  typedef const float __attribute__((address_space(4)))* const_ptr;
  const unsigned long long qa = reinterpret_cast<unsigned long long>(iq_row + h * IDX_D);
  const const_ptr qh = (const_ptr)(((unsigned long long)__builtin_amdgcn_readfirstlane((unsigned)(qa >> 32)) << 32) |
                                   (unsigned)__builtin_amdgcn_readfirstlane((unsigned)qa));
  const float4* src = reinterpret_cast<const float4*>(bk);
  float4 nxt[F4];
  auto fetch = [&](int r0) {
#pragma unroll
    for (int i = 0; i < F4; ++i) {
      const int f = tid + NT * i, j = r0 + (f >> 5);
      nxt[i] = j < n_elig ? src[(long)j * (IDX_D / 4) + (f & 31)] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  fetch(0);
  for (int r0 = 0; r0 < n_elig; r0 += SEQ_RB) {
#pragma unroll
    for (int i = 0; i < F4; ++i) {
      const int f = tid + NT * i;
      *reinterpret_cast<float4*>(stage + (f >> 5) * SEQ_STRIDE + 4 * (f & 31)) = nxt[i];
    }
    __syncthreads();     // the round's rows are staged; the previous round's dsc is consumed
    if (r0 == 0) QM_PHASE(4);
    if (r0 + SEQ_RB < n_elig) fetch(r0 + SEQ_RB);
    const int jr = sub * 64 + lane;
    if (sub < SEQ_RB / 64 && h < idx_heads) {
      // float4 c of the (permuted) row holds elements c / 2 + 16 (4 (c % 2) + t),
      // t < 4: the even ones elements 0..63, the odd ones 64..127
      const float4* row = reinterpret_cast<const float4*>(stage + jr * SEQ_STRIDE);
      float acc = 0.f;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // the half's query elements (scalar loads) and key elements (LDS) are
        // all requested before the first multiply-add: scalar loads complete
        // out of order, so any use of one waits for every LDS read in flight
        float qv[64];
#pragma unroll
        for (int i = 0; i < 64; ++i) qv[i] = qh[64 * half + i];
        float4 kc[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) kc[m] = row[2 * m + half];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int m = 0; m < 16; ++m) {
            const float kv = t == 0 ? kc[m].x : t == 1 ? kc[m].y : t == 2 ? kc[m].z : kc[m].w;
            acc = fmaf(qv[16 * t + m], kv, acc);
          }
      }
      dsc[h][jr] = fmaxf(acc, 0.f);
    }
    __syncthreads();     // dsc complete; every staged row has been read
    if (r0 == 0) QM_PHASE(5);
    if (tid < SEQ_RB && r0 + tid < n_elig) {
      float sc = 0.f;
#pragma unroll
      for (int hh = 0; hh < 4; ++hh)
        if (hh < idx_heads) sc = add_rn(sc, dsc[hh][tid]);
      sc = div_rn(sc, 11.313708498984761f);
      keys[r0 + tid] = sel_key(sc, r0 + tid);
      if (scores_out) scores_out[r0 + tid] = sc;
    }
  }
  const int npad = (n_elig + 31) & ~31;
  for (int j = n_elig + tid; j < npad; j += NT) keys[j] = 0ull;
}

// Top-k of distinct 64-bit keys; sel[rank] = j for rank < topk (rank = the
// number of larger keys). `keys` is padded with zeros (below every real key) to
// a multiple of 32. Up to 128 keys (n <= NT/2), by counting: two adjacent lanes
// split the comparisons of one key and add their counts by DPP. Beyond, by
// a threshold from one histogram over the keys' own range: the upper 32 bits
// (the score) of every key go into 256 equal buckets between their minimum and
// maximum (integer arithmetic, so the bucket is monotone in the key), a suffix
// scan finds the bucket that holds the topk-th largest key, and the keys in it
// and above (typically topk plus a few) are gathered and ranked among
// themselves by counting (1024-thread workgroups; the 256-thread decode
// kernels keep their code small and go straight to radix select). When more
// than RANK_CAND keys share that bucket
// (many equal or clustered scores), radix select instead: eight passes of an
// 8-bit histogram (LDS atomics, then a suffix scan over the 256 digits) pin the
// topk-th largest key T exactly, the keys >= T are gathered, and only they are
// ranked among themselves. `scr` holds rank_scratch(MAXK) ints of LDS;
// topk <= MAXK.
constexpr int rank_scratch(int maxk) { return 256 + 40 + maxk; }
constexpr int RANK_CAND = 128;          // candidates the bucket threshold may leave

// Whole-wave reductions and scans by DPP within rows of 16 lanes and lane
// reads across the four rows (every lane active; results in every lane).
template <int CTRL>
__device__ __forceinline__ unsigned dpp_u(unsigned v) {
  return static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}
template <bool MAX>
__device__ __forceinline__ unsigned wave_minmax_u(unsigned v) {
  auto op = [](unsigned x, unsigned y) { return MAX ? max(x, y) : min(x, y); };
  v = op(v, dpp_u<0xB1>(v));      // quad_perm [1,0,3,2]
  v = op(v, dpp_u<0x4E>(v));      // quad_perm [2,3,0,1]
  v = op(v, dpp_u<0x124>(v));     // row_ror:4
  v = op(v, dpp_u<0x128>(v));     // row_ror:8
  return op(op(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
            op(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
// inclusive prefix sum over the wave's lanes
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += static_cast<int>(dpp_u<0x111>(static_cast<unsigned>(x)));    // row_shr:1
  x += static_cast<int>(dpp_u<0x112>(static_cast<unsigned>(x)));    // row_shr:2
  x += static_cast<int>(dpp_u<0x114>(static_cast<unsigned>(x)));    // row_shr:4
  x += static_cast<int>(dpp_u<0x118>(static_cast<unsigned>(x)));    // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31),
            r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return x + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// The bucket threshold (above). Returns false, having written nothing to sel,
// when more than RANK_CAND keys are at or above the threshold bucket. The
// bucket of a key is ((score bits - min) * mul) >> 32 with width = max - min +
// 1 and mul = 2^40 / width rounded down with a relative margin of 2^-20 (a
// single-precision quotient, whose rounding the margin covers): monotone in the
// key and below 256. Waves exchange partial results through LDS only at the
// four barriers; within a wave, DPP and lane reads.
// Each wave's range of the keys' score bits to wtot (lows, then highs), and
// the histogram and counters cleared: the first pass of bucket_topk, which a
// caller that forms the keys itself (lo / hi over its own keys) runs before
// the barrier that publishes them.
template <int NT>
__device__ __forceinline__ void bucket_range(unsigned lo, unsigned hi, int* scr) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  lo = wave_minmax_u<false>(lo);
  hi = wave_minmax_u<true>(hi);
  if (tid < 256) scr[tid] = 0;             // hist
  if (tid < 8) scr[256 + 32 + tid] = 0;    // state
  if (lane == 0) {
    scr[256 + wv] = static_cast<int>(lo);        // wtot[0..15] lows, [16..31] highs
    scr[256 + 16 + wv] = static_cast<int>(hi);
  }
}

template <int NT>
__device__ bool bucket_topk(const unsigned long long* keys, int n, int topk, int* sel, int* hist, int* wtot,
                            int* state, int* cand, bool range_in) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr int NW = NT / 64;
  static_assert(NW <= 16 && NT >= 256, "wave totals in 16 slots; one bucket per thread");
  if (!range_in) {
    unsigned lo = 0xffffffffu, hi = 0u;
    for (int j = tid; j < n; j += NT) {
      const unsigned v = static_cast<unsigned>(keys[j] >> 32);
      lo = min(lo, v);
      hi = max(hi, v);
    }
    bucket_range<NT>(lo, hi, hist);
    __syncthreads();
  }
  QM_PHASE(6);
  const unsigned glo = wave_minmax_u<false>(lane < NW ? static_cast<unsigned>(wtot[lane]) : 0xffffffffu);
  const unsigned ghi = wave_minmax_u<true>(lane < NW ? static_cast<unsigned>(wtot[16 + lane]) : 0u);
  const float width = static_cast<float>(ghi - glo) + 1.0f;
  const unsigned long long mul =
      static_cast<unsigned long long>(1099511627776.0f * (1.0f - 9.5367431640625e-07f) / width);
  auto bucket = [&](unsigned long long k) {
    return static_cast<int>((static_cast<unsigned long long>(static_cast<unsigned>(k >> 32) - glo) * mul) >> 32);
  };
  for (int j = tid; j < n; j += NT) atomicAdd(&hist[bucket(keys[j])], 1);
  __syncthreads();                        // every wave has read the range: wtot is free
  QM_PHASE(7);
  // suffix sums over the buckets in one wave (no exchange of wave totals):
  // lane l takes buckets 255 - 4 l .. 252 - 4 l, the keys above them are the
  // exclusive scan of the lanes' sums, then the lane walks its four downwards
  if (wv == 0) {
    const int4 hv = *reinterpret_cast<const int4*>(&hist[252 - 4 * lane]);
    const int s4 = (hv.x + hv.y) + (hv.z + hv.w);
    int above = wave_incl_sum(s4) - s4;
    const int hb[4] = {hv.w, hv.z, hv.y, hv.x};     // buckets 255 - 4 l - i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int incl = above + hb[i];
      if (above < topk && incl >= topk) {    // the bucket of the topk-th largest key
        state[0] = 255 - 4 * lane - i;
        state[1] = incl;                     // keys in it and above
      }
      above = incl;
    }
  }
  __syncthreads();
  QM_PHASE(8);
  const int bstar = state[0], n_cand = state[1];
#ifdef QM_PHASE_TRACE
  if (threadIdx.x == 0) qm_ph_[14] = static_cast<unsigned long long>(n_cand);
#endif
  if (n_cand > RANK_CAND) return false;
  // gather, in any order (the ranks below do not depend on it): one LDS atomic
  // per wave reserves the wave's places, lanes take theirs by mask count. The
  // keys go where the histogram was, zero-padded to a multiple of 32.
  unsigned long long* ckey = reinterpret_cast<unsigned long long*>(hist);
  const int cpad = (n_cand + 31) & ~31;
  for (int c = n_cand + tid; c < cpad; c += NT) ckey[c] = 0ull;
  for (int j0 = 0; j0 < n; j0 += NT) {
    const int j = j0 + tid;
    const unsigned long long k = j < n ? keys[j] : 0ull;
    const bool pick = j < n && bucket(k) >= bstar;
    const unsigned long long m = __ballot(pick);
    int base = 0;
    if (lane == 0 && m) base = atomicAdd(&state[2], __popcll(m));
    base = __builtin_amdgcn_readfirstlane(base);
    if (pick) {
      const int at = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(m >> 32),
                                                                      __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(m), 0u)));
      ckey[at] = k;
      cand[at] = j;
    }
  }
  __syncthreads();
  QM_PHASE(9);
  // rank by counting: two adjacent lanes split one candidate's comparisons
  // (only the waves that hold candidates)
  if (tid < 2 * cpad) {
    const int c = tid >> 1, part = tid & 1, hc = cpad >> 1;
    const unsigned long long kc = ckey[c < n_cand ? c : 0];
    int rank = 0;
    for (int i = part * hc; i < part * hc + hc; i += 16) {
      unsigned long long k16[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) k16[u] = ckey[i + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) rank += k16[u] > kc ? 1 : 0;
    }
    rank += __builtin_amdgcn_update_dpp(0, rank, 0xB1, 0xF, 0xF, true);
    if (part == 0 && c < n_cand && rank < topk) sel[rank] = cand[c];
  }
  return true;
}

// range_in: the caller ran bucket_range<NT> over all n keys behind the
// barrier that published them (used only when the bucket threshold runs)
template <int NT, int MAXK>
__device__ void rank_topk(const unsigned long long* keys, int n, int topk, int* sel, int* scr,
                          bool range_in = false) {
  static_assert(NT >= 256 && NT % 64 == 0 && NT <= 1024, "one digit per thread");
  const int tid = threadIdx.x;
  const int npad = (n + 31) & ~31;
  if (n <= NT / 2 && n <= 128) {
    const int j = tid >> 1, part = tid & 1, half = npad >> 1;
    const unsigned long long kj = keys[j < n ? j : 0];
    int rank = 0;
    for (int i = part * half; i < part * half + half; i += 16) {
      unsigned long long k16[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) k16[u] = keys[i + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) rank += k16[u] > kj ? 1 : 0;
    }
    rank += __builtin_amdgcn_update_dpp(0, rank, 0xB1, 0xF, 0xF, true);
    if (part == 0 && j < n && rank < topk) sel[rank] = j;
    return;
  }
  int* hist = scr;                        // [256]
  int* wtot = scr + 256;                  // [16]
  int* state = scr + 256 + 32;            // prefix lo, prefix hi, remaining, count
  int* cand = scr + 256 + 40;             // [topk]
  const int lane = tid & 63, wv = tid >> 6;
  if constexpr (NT >= 1024)
    if (topk <= RANK_CAND && bucket_topk<NT>(keys, n, topk, sel, hist, wtot, state, cand, range_in)) return;
  unsigned long long prefix = 0ull;
  int r = topk;
  for (int shift = 56; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int j = tid; j < n; j += NT) {
      const unsigned long long k = keys[j];
      const bool match = shift == 56 || ((k ^ prefix) >> (shift + 8)) == 0ull;
      if (match) atomicAdd(&hist[(k >> shift) & 255], 1);
    }
    __syncthreads();
    // suffix sums over the digits: thread t takes digit 255 - t
    int h = 0, incl = 0;
    if (tid < 256) {
      h = hist[255 - tid];
      incl = h;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int x = __shfl_up(incl, o, 64);
        if (lane >= o) incl += x;
      }
      if (lane == 63) wtot[wv] = incl;
    }
    __syncthreads();
    if (tid < 256) {
      for (int w = 0; w < wv; ++w) incl += wtot[w];
      const int above = incl - h;          // keys of the prefix with a larger digit
      if (above < r && incl >= r) {
        const unsigned long long np = prefix | (static_cast<unsigned long long>(255 - tid) << shift);
        state[0] = static_cast<int>(np & 0xffffffffull);
        state[1] = static_cast<int>(np >> 32);
        state[2] = r - above;
      }
    }
    __syncthreads();
    prefix = (static_cast<unsigned long long>(static_cast<unsigned>(state[1])) << 32) |
             static_cast<unsigned>(state[0]);
    r = state[2];
  }
  // prefix is now the topk-th largest key: gather the keys >= it, then rank them
  if (tid == 0) state[3] = 0;
  __syncthreads();
  for (int j = tid; j < n; j += NT)
    if (keys[j] >= prefix) cand[atomicAdd(&state[3], 1)] = j;
  __syncthreads();
  for (int c = tid; c < topk; c += NT) {
    const unsigned long long kc = keys[cand[c]];
    int rank = 0;
    for (int i = 0; i < topk; ++i) rank += keys[cand[i]] > kc ? 1 : 0;
    sel[rank] = cand[c];
  }
}

// File one selected entry: row s of sequence b took block j as its slot-th selection.
__device__ __forceinline__ void file_entry(uint16_t* tab, int b, int max_blocks, int seq, int j, int s, int slot) {
  tab[((long)b * max_blocks + j) * seq + s] = static_cast<uint16_t>(slot + 1);
}

// The (max, sum) pairs of a row's slot that holds no partial.
__device__ __forceinline__ void empty_partial(float* part_ml, long row, int hkv, int nslot, int slot) {
  for (int g = 0; g < hkv; ++g) {
    float4* ml = reinterpret_cast<float4*>(part_ml + (((long)row * hkv + g) * nslot + slot) * GQA * 2);
#pragma unroll
    for (int h = 0; h < GQA / 2; ++h) ml[h] = make_float4(-INFINITY, 0.f, -INFINITY, 0.f);
  }
}

struct SelArgs {
  const float* iq; const float* block_keys; const int* positions; const int* page_table;
  int* ids; int* n_sel; int2* items; float* scores_out;
  int batch, seq, idx_heads, ratio, topk, max_blocks, page_size, max_pages, max_items;
  // the chunk path's slot table (qm_qsa_select_chunk files into it), or null
  uint16_t* tab = nullptr; float* part_ml = nullptr;
  int hkv = 0;
  // the rows' block scores from qsa_score_rows_kernel ([row][max_blocks]), or
  // null when the selection scores the blocks itself
  const float* scores_in = nullptr;
};

struct SelShared {
  float q[4 * IDX_D];
  float dsc[4][SELP_NT / 4];            // a scoring round's relu'd dot products (several-rows order)
  float newkey[IDX_D];
  unsigned long long key[SEL_MAX_BLOCKS];
  int pages[SEL_MAX_BLOCKS];
  int sel[SEL_MAX_BLOCKS / 2];
  alignas(16) int rscr[rank_scratch(SEL_MAX_BLOCKS / 2)];
};

// Selection for one query row at position p, by a whole SEL_NT-thread block.
// The indexer query must already be in S.q (heads past idx_heads zero). Block
// keys come from the cache, except block new_j (>= 0 when this very launch
// completed it), whose key is in S.newkey.
template <int NT>
__device__ void select_row(const SelArgs& A, SelShared& S, int row, int b, int p, int new_j, float* stage) {
  const int tid = threadIdx.x;
  const int n_elig = min((p + 1) / A.ratio, A.max_blocks);
  const int n_sel = min(n_elig, A.topk);
  int* out_ids = A.ids + (long)row * A.topk;

  // the page-table row, needed to describe the attention items, comes in with the keys
  const int n_lpages = min(A.max_pages, (p + A.page_size) / A.page_size);
  if (A.items)
    for (int i = tid; i < n_lpages; i += NT) S.pages[i] = A.page_table[(long)b * A.max_pages + i];
  if (A.scores_out)
    for (int j = tid; j < A.max_blocks; j += NT)
      if (j >= n_elig) A.scores_out[(long)row * A.max_blocks + j] = -INFINITY;

  bool range_in = false;
  if (A.scores_in) {
    if (n_elig > A.topk) {
      const float* sc = A.scores_in + (long)row * A.max_blocks;
      unsigned lo = 0xffffffffu, hi = 0u;
      for (int j = tid; j < n_elig; j += NT) {
        const unsigned long long k = sel_key(sc[j], j);
        S.key[j] = k;
        lo = min(lo, static_cast<unsigned>(k >> 32));
        hi = max(hi, static_cast<unsigned>(k >> 32));
      }
      const int npad = (n_elig + 31) & ~31;
      for (int j = n_elig + tid; j < npad; j += NT) S.key[j] = 0ull;
      // the bucket threshold's key range, published by the barrier below
      if constexpr (NT >= 1024) {
        bucket_range<NT>(lo, hi, S.rscr);
        range_in = true;
      }
    }
  } else if (n_elig > A.topk || A.scores_out) {
    const float* bk = A.block_keys + (long)b * A.max_blocks * IDX_D;
    float* sc_out = A.scores_out ? A.scores_out + (long)row * A.max_blocks : nullptr;
    if (NT != SELP_NT || A.seq == 1) {
      // one query row (the 256-thread front kernel serves decode only): the
      // first passes of block keys are in flight across the barrier
      float kp[score_pre<NT>()][8];
      prefetch_block_keys<NT>(kp, bk, n_elig, new_j, true);
      __syncthreads();    // S.q and S.newkey visible
      score_blocks<NT>(S.q, S.newkey, bk, n_elig, new_j, A.idx_heads, S.key, sc_out, kp);
    } else {
      // several rows (a block completed in this call is already in the cache)
      if constexpr (NT == SELP_NT)
        score_blocks_seq<NT>(A.iq + (long)row * A.idx_heads * IDX_D, bk, n_elig, A.idx_heads, S.key, sc_out,
                             S.dsc, stage);
    }
  }
  __syncthreads();
  QM_PHASE(1);
  if (n_elig <= A.topk) {
    for (int i = tid; i < n_elig; i += NT) { out_ids[i] = i; S.sel[i] = i; }
  } else {
    rank_topk<NT, SEL_MAX_BLOCKS / 2>(S.key, n_elig, A.topk, S.sel, S.rscr, range_in);
    __syncthreads();
    QM_PHASE(2);
    for (int i = tid; i < A.topk; i += NT) out_ids[i] = S.sel[i];
  }
  if (tid == 0) A.n_sel[row] = n_sel;
  if (A.tab) {
    // the chunk path's slot table, as qsa_chunk_bucket_kernel fills it: every
    // selected block files the row's slot, and the slots this row leaves
    // empty get (max, sum) = (-inf, 0)
    __syncthreads();
    const int s = row % A.seq;
    const int nslot = A.topk + 1;
    for (int i = tid; i < nslot; i += NT) {
      bool empty;
      if (i < A.topk) {
        empty = i >= n_sel;
        if (!empty) file_entry(A.tab, b, A.max_blocks, A.seq, S.sel[i], s, i);
      } else {
        empty = ((p + 1) / A.ratio) * A.ratio > p;      // the row completes its block: no tail
      }
      if (empty) empty_partial(A.part_ml, row, A.hkv, nslot, i);
    }
  }
  if (!A.items) return;
  __syncthreads();
  // attention items: the groups of every selected block in rank order, then the tail's
  int2* items = A.items + (long)row * A.max_items;
  const int gpb = A.ratio >= 32 ? A.ratio / 32 : 1;
  const int n_blk_items = n_sel * gpb;
  const int ts = ((p + 1) / A.ratio) * A.ratio;
  const int n_tail = ts > p ? 0 : (p >> 5) - (ts >> 5) + 1;
  const int n_items = n_blk_items + n_tail;
  for (int it = tid; it < n_items; it += NT) {
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

// Block scores of the query rows of a chunk (several rows per sequence) in the
// reference's several-rows summation order: one fused multiply-add chain over
// the 128 elements per (row, block, head), then relu, the heads added in order
// and the division by sqrt(128), as score_blocks_seq forms them. Workgroup
// (tile of 64 blocks, 4 rows, sequence): the tile's block rows are staged in
// LDS with coalesced loads (rows padded by 16 bytes, so that the lanes' row
// reads fall on distinct banks); wave w takes row 4 y + w and lane l block
// 64 x + l, running the idx_heads chains side by side (each key element read
// once feeds every head); the 4 query rows are staged in LDS beside the block
// rows. Scores past a row's eligible blocks are -inf when `fill` is set and
// left unwritten otherwise.
constexpr int SCR_BLK = 64;                 // blocks per workgroup, one per lane
constexpr int SCR_ROWS = 4;                 // query rows per workgroup, one per wave
constexpr int SCR_STRIDE = IDX_D / 4 + 1;   // float4 per staged block row

struct ScoreRowsArgs {
  const float* iq; const float* block_keys; const int* positions; float* scores;
  int seq, idx_heads, ratio, max_blocks;
  int fill;
};

__global__ __launch_bounds__(64 * SCR_ROWS) void qsa_score_rows_kernel(ScoreRowsArgs A) {
  __shared__ float4 rows_lds[SCR_BLK * SCR_STRIDE];
  __shared__ float4 q_lds[SCR_ROWS][IDX_D];      // 4 heads x 128 per row, zeros past idx_heads
  const int b = blockIdx.z, tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j0 = blockIdx.x * SCR_BLK, s0 = blockIdx.y * SCR_ROWS;
  // the position by a vector load issued first, then the tile's block rows
  // and the group's query rows before it is known (block rows clamped to the
  // cache's max_blocks, query rows to the sequence, so that every load is
  // in bounds and none waits behind the position); the zeros past the
  // eligible blocks and the group's rows are applied after
  const unsigned pos_raw = __builtin_amdgcn_raw_buffer_load_b32(dev_rsrc(A.positions + b, 4), 0, 0, 0);
  const float4* src = reinterpret_cast<const float4*>(A.block_keys + (long)b * A.max_blocks * IDX_D);
  const float4* qsrc = reinterpret_cast<const float4*>(A.iq + (long)b * A.seq * A.idx_heads * IDX_D);
  constexpr int F4 = SCR_BLK * IDX_D / 4 / (64 * SCR_ROWS);
  const int q4 = A.idx_heads * IDX_D / 4;     // float4 per query row
  float4 kv[F4], qv[SCR_ROWS];
#pragma unroll
  for (int i = 0; i < F4; ++i) {
    const int f = tid + 64 * SCR_ROWS * i;
    kv[i] = src[(long)min(j0 + (f >> 5), A.max_blocks - 1) * (IDX_D / 4) + (f & 31)];
  }
  // the group's query rows: thread t < 128 takes float4 t of each row's
  // idx_heads x 128 (zeros past them)
#pragma unroll
  for (int r = 0; r < SCR_ROWS; ++r) qv[r] = qsrc[(long)min(s0 + r, A.seq - 1) * q4 + min(tid, q4 - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const int pos0 = __builtin_amdgcn_readfirstlane((int)pos_raw);
  const int s_last = min(s0 + SCR_ROWS, A.seq) - 1;
  const int elig_max = min((pos0 + s_last + 1) / A.ratio, A.max_blocks);   // the group's last row sees the most
  const int s = s0 + wv, j = j0 + lane;
  float* out = A.scores + ((long)b * A.seq + s) * A.max_blocks;
  if (j0 >= elig_max) {
    // no row of the group has an eligible block in this tile
    if (A.fill && s < A.seq && j < A.max_blocks) out[j] = -INFINITY;
    return;
  }
#pragma unroll
  for (int i = 0; i < F4; ++i)
    if (j0 + ((tid + 64 * SCR_ROWS * i) >> 5) >= elig_max) kv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < SCR_ROWS; ++r)
    if (s0 + r >= A.seq || tid >= q4) qv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < F4; ++i) {
    const int f = tid + 64 * SCR_ROWS * i;
    rows_lds[(f >> 5) * SCR_STRIDE + (f & 31)] = kv[i];
  }
  if (tid < IDX_D)
#pragma unroll
    for (int r = 0; r < SCR_ROWS; ++r) q_lds[r][tid] = qv[r];
  __syncthreads();
  if (s >= A.seq) return;
  const int n_elig = min((pos0 + s + 1) / A.ratio, A.max_blocks);
  const int nh = A.idx_heads;
  const float4* row = &rows_lds[lane * SCR_STRIDE];
  const float* qrow = reinterpret_cast<const float*>(&q_lds[wv][0]);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    // float4 c of the (permuted) row holds elements c / 2 + 16 (4 (c % 2) + t),
    // t < 4: the even ones elements 0..63, the odd ones 64..127
    float4 kc[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) kc[m] = row[2 * m + half];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // elements d = 64 half + 16 t + m, m < 16, in order; the step's query
      // elements come from LDS at one address per wave (a broadcast), all
      // requested before the step's first multiply-add. Heads past idx_heads
      // multiply the staged zeros and stay out of the sum (a condition on the
      // head count inside the loops would have the compiler copy them per count).
      float4 qv4[4][4];
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int m4 = 0; m4 < 4; ++m4)
          qv4[h][m4] = *reinterpret_cast<const float4*>(qrow + h * IDX_D + 64 * half + 16 * t + 4 * m4);
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const float kvv = t == 0 ? kc[m].x : t == 1 ? kc[m].y : t == 2 ? kc[m].z : kc[m].w;
        const int e = m & 3;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float4 q4 = qv4[h][m >> 2];
          acc[h] = fmaf(e == 0 ? q4.x : e == 1 ? q4.y : e == 2 ? q4.z : q4.w, kvv, acc[h]);
        }
      }
      // the step's products complete here and the next step's reads stay
      // behind them (an empty asm that takes the sums and clobbers memory):
      // requested all at once, the reads would need registers for every step,
      // and the other waves of the SIMD cover their latency
      asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]) : : "memory");
    }
  }
  float sc = 0.f;
#pragma unroll
  for (int h = 0; h < 4; ++h)
    if (h < nh) sc = add_rn(sc, fmaxf(acc[h], 0.f));
  sc = div_rn(sc, 11.313708498984761f);
  if (j < n_elig) out[j] = sc;
  else if (A.fill && j < A.max_blocks) out[j] = -INFINITY;
}

// Block scores of one query row per sequence (decode) in the reference's
// one-row summation order (row16_block_score, the order of the front and
// decode kernels), spread over the blocks: workgroup (64 blocks, sequence),
// 16 lanes per block, the 4 passes' key loads all issued before the first
// product. Scores past the row's eligible blocks are -inf (up to max_blocks).
constexpr int SC1_BLK = 64;                    // blocks per workgroup
constexpr int SC1_NT = 256;

struct ScoreRowArgs {
  const float* iq; const float* block_keys; const int* positions; float* scores;
  int idx_heads, ratio, max_blocks;
};

__global__ __launch_bounds__(SC1_NT) void qsa_score_row_kernel(ScoreRowArgs A) {
  constexpr int PASS = SC1_NT / SCORE_LANES;   // blocks per pass: 16
  constexpr int NPASS = SC1_BLK / PASS;        // 4
  const int b = blockIdx.y, tid = threadIdx.x, m = tid & 15, jl = tid >> 4;
  const int j0 = blockIdx.x * SC1_BLK;
  const int n_elig = min((A.positions[b] + 1) / A.ratio, A.max_blocks);
  float* out = A.scores + (long)b * A.max_blocks;
  if (j0 >= n_elig) {
    for (int j = j0 + tid; j < min(j0 + SC1_BLK, A.max_blocks); j += SC1_NT) out[j] = -INFINITY;
    return;
  }
  const float* bk = A.block_keys + (long)b * A.max_blocks * IDX_D;
  float kp[NPASS][8];
#pragma unroll
  for (int u = 0; u < NPASS; ++u) {
    const int j = j0 + u * PASS + jl;
    load_block_part(kp[u], bk, j, j < n_elig);
  }
  // this lane's elements 16 i + m of the 4 query rows (heads past idx_heads zero)
  const float* q_row = A.iq + (long)b * A.idx_heads * IDX_D;
  float q[4][8];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) q[h][i] = h < A.idx_heads ? q_row[h * IDX_D + 16 * i + m] : 0.f;
#pragma unroll
  for (int u = 0; u < NPASS; ++u) {
    const int j = j0 + u * PASS + jl;
    const float sc = row16_block_score(q, kp[u], A.idx_heads);
    if (m == 0 && j < A.max_blocks) out[j] = j < n_elig ? sc : -INFINITY;
  }
}

__global__ __launch_bounds__(SELP_NT) void qsa_select_kernel(SelArgs A) {
  QM_PHASE_DECL
  const int row = blockIdx.x;
  const int b = row / A.seq, s = row % A.seq;
  const int p = A.positions[b] + s;
  __shared__ SelShared S;
  QM_PHASE(0);
  for (int i = threadIdx.x; i < 4 * IDX_D; i += SELP_NT)
    S.q[i] = i < A.idx_heads * IDX_D ? A.iq[(long)row * A.idx_heads * IDX_D + i] : 0.f;
  __syncthreads();
  __shared__ float4 stage[SEQ_STAGE / 4];   // block rows of a scoring round (several rows per sequence)
  select_row<SELP_NT>(A, S, row, b, p, -1, reinterpret_cast<float*>(stage));
  QM_PHASE(3);
  QM_PHASE_FLUSH();
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
    if (threadIdx.x < 64) prep_wave<T>(A, b, role);
    return;
  }
  const int tid = threadIdx.x;
  const int p = A.positions[b];
  __shared__ SelShared S;
  __shared__ float s_x[QSA_D], s_y[QSA_D], s_scr[32];
  if (tid < IDX_D) A.raw_keys[((long)b * A.max_ctx + p) * IDX_D + tid] = A.ik[(long)b * IDX_D + tid];
  const float2 csv = rope_cs(A.cos, A.sin, p, A.rope);
  for (int h = 0; h < 4; ++h) {
    __syncthreads();
    if (h >= A.idx_heads) {
      if (tid < IDX_D) S.q[h * IDX_D + tid] = 0.f;
      continue;
    }
    if (tid < IDX_D) s_x[tid] = Act<T>::load(A.iq, ((long)b * A.idx_heads + h) * IDX_D + tid);
    const float y = norm_rope_row<T>(s_x, s_y, s_scr, IDX_D, A.iq_norm, A.eps, A.rope, csv.x, csv.y);
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
  select_row<SEL_NT>(SA, S, b, b, p, new_j, nullptr);
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
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
    const uint16_t* qh = A.q + q_index(row, A.hkv, 0, hq, 8 * quad);
    const uint16_t* ql = A.q + q_index(row, A.hkv, 1, hq, 8 * quad);
    const bf16x8_t zero = {};
#pragma unroll
    for (int sk = 0; sk < 8; ++sk) {
      qhi[sk] = col < GQA ? load_bf16x8(qh + Q_SK_STRIDE * sk) : zero;
      qlo[sk] = col < GQA ? load_bf16x8(ql + Q_SK_STRIDE * sk) : zero;
    }
  }

  f32x4_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  if (item < n_items) {
    const int page = desc.x / A.page_size, row0 = desc.x % A.page_size;
    const int lo = desc.y & 0xff, hi = desc.y >> 8;
    const long pbase = ((long)page * A.hkv + g) * A.page_size * QSA_D;
    const uint16_t* kp = A.k_pool + pbase + (row0 >> 4) * 8 * 512 + lane * 8;
    const uint16_t* vp = A.v_pool + pbase + (row0 >> 5) * 16 * 512 + lane * 8;
    bf16x8_t kf[2][8], vf[16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int sk = 0; sk < 8; ++sk) kf[t][sk] = load_bf16x8(kp + (t * 8 + sk) * 512);
#pragma unroll
    for (int db = 0; db < 16; ++db) vf[db] = load_bf16x8(vp + db * 512);

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

// Partial outputs are either fp32 and unnormalised (o = sum p v) or bf16 and
// normalised by their own sum (o / l, the chunk path's 16-bit partials).
template <typename T, typename PO = float>
struct CombineArgs {
  const PO* part_o; const float* part_ml; const T* qg; T* out;
  int hq, hkv, splits;
  // the chunk path's slot table, cleared here once the attention has read
  // it: its length in 16-byte words
  uint16_t* tab = nullptr;
  long tab_words = 0;
};

__device__ __forceinline__ float part_value(const float* p, long i) { return p[i]; }
__device__ __forceinline__ float part_value(const uint16_t* p, long i) { return bf16_to_f32(p[i]); }

constexpr int MAX_SPLITS = 1024;

template <typename T, typename PO = float>
__global__ __launch_bounds__(QSA_D) void qsa_combine_kernel(CombineArgs<T, PO> A) {
  constexpr bool normed = sizeof(PO) == 2;
  const int hq = blockIdx.x, row = blockIdx.y;
  const int d = threadIdx.x;
  const int g = hq / GQA, hh = hq % GQA;
  const long base = (((long)row * A.hkv + g) * A.splits) * GQA + hh;
  __shared__ float s_w[MAX_SPLITS];
  __shared__ float s_red[QSA_D / 64];
  const float gate = Act<T>::load(A.qg, ((long)row * A.hq + hq) * (2 * QSA_D) + QSA_D + d);
  if (A.tab) {
    // each workgroup clears 4 KB stretches of the table, spread over the grid
    const long wg = blockIdx.x + (long)gridDim.x * blockIdx.y, n_wg = (long)gridDim.x * gridDim.y;
    for (long w = wg * QSA_D + d; w < A.tab_words; w += n_wg * QSA_D)
      reinterpret_cast<u32x4_t*>(A.tab)[w] = u32x4_t{0u, 0u, 0u, 0u};
  }
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
    const float lw = A.part_ml[(base + (long)s * GQA) * 2 + 1] * w;
    l += lw;
    s_w[s] = normed ? lw : w;
  }
  l = wave_sum(l);
  __syncthreads();
  if ((d & 63) == 0) s_red[d >> 6] = l;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int i = 0; i < QSA_D / 64; ++i) L += s_red[i];
  float o = 0.f;
  // loads are unconditional so that eight are in flight at once; a slot of
  // zero weight (never written, or under the max by ~88) adds exactly 0
#pragma unroll 8
  for (int s = 0; s < A.splits; ++s) {
    const float v = part_value(A.part_o, (base + (long)s * GQA) * QSA_D + d);
    o += s_w[s] != 0.f ? v * s_w[s] : 0.f;
  }
  const float att = Act<T>::round(o / L);
  const float sg = Act<T>::round(sigmoid_f(gate));
  Act<T>::store(A.out, ((long)row * A.hq + hq) * QSA_D + d, att * sg);
}

// ---------------------------------------------------------------------------
// chunk attention (prefill), block-major
// ---------------------------------------------------------------------------
// The attention of a chunk of query rows reads each key/value block once. A
// row's entries are its (row, slot) pairs: slot i < n_sel its i-th selected
// block, slot topk its tail block (keys ts..p, when the row does not complete
// its block). The entries are filed in a slot table, [B][max_blocks][seq]
// uint16 in the workspace: entry (b, j, s) holds slot + 1 when row s selected
// block j, else 0. Plain stores fill it (no atomics, so no round trip holds up
// the filing), the attention reads a block's row of it, and the merge clears
// it, so every call leaves the table zero. qm_qsa_attend_chunk is three
// launches:
//   qsa_chunk_bucket   one 64-thread workgroup per row: files the row's
//                      selected entries and writes the empty partials (max
//                      -inf) of its unused slots (qm_qsa_select_chunk does the
//                      same inside the selection);
//   qsa_chunk_attend   grid (blocks + tail workgroups, kv head, sequence): the
//                      workgroup of block j reads its table row and the page
//                      with its first loads, then the block's 64 tokens of key
//                      pieces straight into LDS (16 KB per 32 tokens) and of
//                      value pieces into registers; each wave scores two
//                      entries x 8 query heads on bf16 MFMA and writes one
//                      partial per (row, slot, head): fp32 max and sum, and the
//                      output normalised by the sum, in bf16. Every wave finds
//                      the entries it needs from the table row by ballot, so
//                      the workgroup's LDS is the keys and the softmax weights
//                      alone (40 KB: four workgroups per compute unit). A tail
//                      workgroup takes the tail entries of 8 rows (one or two
//                      blocks), which would otherwise pile onto two blocks'
//                      workgroups;
//   qsa_combine        merges a row's topk + 1 slots, applies the gate and
//                      clears the slot table.
// The workspace is zero-filled before its first use; the selection (or the
// bucket kernel) and the attention of one call use the same seq.
constexpr int CA_MAX_BLOCKS = 4096;
constexpr int CA_NT = 256;        // attention workgroup: four waves
constexpr int CA_TAIL_ROWS = 8;   // rows per tail workgroup

struct ChunkAttnArgs {
  const uint16_t* q;                      // [rows, 2 (hi, lo), hq, 256] bf16
  const uint16_t* k_pool; const uint16_t* v_pool;
  const int* positions; const int* page_table;
  uint16_t* part_o; float* part_ml;      // part_o: bf16, normalised by l
  const uint16_t* tab;                    // [B][max_blocks][seq]: slot + 1, or 0
  int batch, seq, hq, hkv, page_size, max_pages, ratio, topk, max_blocks, nwg_sel;
  float scale;
};

struct ChunkBucketArgs {
  const int* positions; const int* ids; const int* n_sel;
  float* part_ml; uint16_t* tab;
  int batch, seq, hkv, ratio, topk, max_blocks;
};

__global__ __launch_bounds__(64) void qsa_chunk_bucket_kernel(ChunkBucketArgs A) {
  const int row = blockIdx.x, lane = threadIdx.x;
  const int b = row / A.seq, s = row % A.seq;
  const int nslot = A.topk + 1;
  const int nsel = A.n_sel[row];
  const int p = A.positions[b] + s;
  for (int i = lane; i < nslot; i += 64) {
    bool empty;
    if (i < A.topk) {
      empty = i >= nsel;
      if (!empty) file_entry(A.tab, b, A.max_blocks, A.seq, A.ids[(long)row * A.topk + i], s, i);
    } else {
      empty = ((p + 1) / A.ratio) * A.ratio > p;      // the row completes its block: no tail
    }
    if (empty) empty_partial(A.part_ml, row, A.hkv, nslot, i);
  }
}

// Workgroup LDS of the chunk attention: the block's keys and the softmax
// weights every wave hands to the others.
struct ChunkShared {
  uint16_t k[2][16][64 * 8];     // per 32-token group: 16 key pieces of 1 KB (16 tokens x 32 channels)
  bf16x8_t p[2][4][64];          // softmax weights / sum: [group][column block = wave that formed it][lane]
};
static_assert(sizeof(ChunkShared) == 40960, "four workgroups per compute unit");

// The next 8 entries of a 128-row span of a block's table row, in row order:
// lane l holds rows (span base + l) and (span base + 64 + l) as `ma` / `mb` =
// row << 16 | slot, and `ra` / `rb` are the rows of the span not yet taken
// (bit l: lane l's row is an entry). Scalar work: the first set bits, read out
// of their lanes; entry 2 cw + odd goes to pko[cw] of the lanes of that
// parity. Entries past the span's last repeat the group's first.
__device__ __forceinline__ void next_group(unsigned long long& ra, unsigned long long& rb, unsigned ma, unsigned mb,
                                           bool odd, unsigned (&pko)[4]) {
  unsigned first = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    unsigned v;
    if (ra != 0ull) {
      v = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(ma), __builtin_ctzll(ra)));
      ra &= ra - 1ull;
    } else if (rb != 0ull) {
      v = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(mb), __builtin_ctzll(rb)));
      rb &= rb - 1ull;
    } else {
      v = first;
    }
    if (i == 0) first = v;
    if ((i & 1) == 0) pko[i >> 1] = v;
    else pko[i >> 1] = odd ? v : pko[i >> 1];
  }
}

// pko[w] for a wave-uniform w
__device__ __forceinline__ unsigned pick4(const unsigned (&v)[4], int w) {
  return w == 0 ? v[0] : w == 1 ? v[1] : w == 2 ? v[2] : v[3];
}

// Where a column's partial row goes: entry pk (row << 16 | tail << 9 | slot), query head hh.
__device__ __forceinline__ long chunk_partial_row(const ChunkAttnArgs& A, unsigned pk, long row_b, int g, int nslot,
                                                  int hh) {
  return (((row_b + (pk >> 16)) * A.hkv + g) * nslot + (pk & 511)) * GQA + hh;
}

// One wave's scores over the block for its two entries x 8 query heads (lane
// column il = which entry, hh = query head): the softmax weights of its 16
// columns, divided by their sums, go to S.p as the PV product's operands; the
// (max, sum) pairs go to the workspace.
__device__ __forceinline__ void chunk_scores(const ChunkAttnArgs& A, ChunkShared& S, const bf16x8_t (&qhi)[8],
                                             int j, unsigned pk, bool ok, long row_b, int pos0, int g, int nslot,
                                             bool mark = false) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, quad = lane >> 4, col = lane & 15, hh = lane & 7;
  const int gpb = A.ratio / 32;
  const bool tail = (pk >> 9) & 1u;
  const int p = pos0 + static_cast<int>(pk >> 16);
  // a tile's key fragments are read from LDS four at a time before their
  // products, so that their latencies overlap (eight at a time would not
  // leave registers for four waves per SIMD)
  f32x4_t sc[2][2];
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
      if (gi < gpb) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          bf16x8_t kf[4];
#pragma unroll
          for (int u = 0; u < 4; ++u)
            kf[u] = *reinterpret_cast<const bf16x8_t*>(&S.k[gi][t * 8 + 4 * h + u][lane * 8]);
#pragma unroll
          for (int u = 0; u < 4; ++u) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[u], qhi[4 * h + u], c, 0, 0, 0);
        }
      }
      sc[gi][t] = c;
    }
  }
  // keys of a tail entry stop at the row's own position: key gi*32 + 16t +
  // 4quad + v of the block is visible when gi*32 + 16t + v <= lim
  const int lim = !ok ? -1 : tail ? p - j * A.ratio - 4 * quad : 1 << 20;
  float mx = -INFINITY;
#pragma unroll
  for (int gi = 0; gi < 2; ++gi)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float xs = (gi < gpb && gi * 32 + 16 * t + v <= lim) ? sc[gi][t][v] * A.scale : -INFINITY;
        sc[gi][t][v] = xs;
        mx = fmaxf(mx, xs);
      }
  mx = xor32_max(xor16_max(mx));
  if (mark) QM_PHASE(9);
  float lsum = 0.f;
#pragma unroll
  for (int gi = 0; gi < 2; ++gi)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float e = sc[gi][t][v] == -INFINITY ? 0.f : __expf(sc[gi][t][v] - mx);
        sc[gi][t][v] = e;
        lsum += e;
      }
  const float l = xor32_sum(xor16_sum(lsum));
  // a column of no entry has l = 0: its weights are 0
  const float rl = ok ? 1.0f / l : 0.f;
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    unsigned pw[4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      pw[2 * t] = pack_bf16x2(sc[gi][t][0] * rl, sc[gi][t][1] * rl);
      pw[2 * t + 1] = pack_bf16x2(sc[gi][t][2] * rl, sc[gi][t][3] * rl);
    }
    S.p[gi][wv][lane] = __builtin_bit_cast(bf16x8_t, u32x4_t{pw[0], pw[1], pw[2], pw[3]});
  }
  if (mark) QM_PHASE(10);
  if (quad == 0 && ok)
    *reinterpret_cast<float2*>(A.part_ml + chunk_partial_row(A, pk, row_b, g, nslot, hh) * 2) = make_float2(mx, l);
  (void)col;
}

// A wave with no entry in the group: its columns' weights are zero.
__device__ __forceinline__ void chunk_no_scores(ChunkShared& S) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const bf16x8_t zero = __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
  S.p[0][wv][lane] = zero;
  S.p[1][wv][lane] = zero;
}

// The outputs of a group's 64 columns (4 waves' entries x 8 query heads) in
// this wave's 64 channels (64 wv ..: value blocks 4 wv .. 4 wv + 3, whose
// pieces `vr` the wave holds), written straight from the product's lanes
// (two 16-byte stores per lane and column block, each of the four quads'
// stores together 64 contiguous bytes of a partial row). pko/oko: the entries
// of column block cw's lanes (entry il of wave cw) and whether they exist.
__device__ __forceinline__ void chunk_outputs(const ChunkAttnArgs& A, ChunkShared& S, const bf16x8_t (&vr)[2][4],
                                              const unsigned (&pko)[4], const bool (&oko)[4], long row_b, int g,
                                              int nslot, bool mark = false) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, quad = lane >> 4, hh = lane & 7;
  const int gpb = A.ratio / 32;
#pragma unroll
  for (int cw = 0; cw < 4; ++cw) {
    f32x4_t acc[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
      if (gi < gpb) {
        const bf16x8_t pf = S.p[gi][cw][lane];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vr[gi][cb], pf, acc[cb], 0, 0, 0);
      }
    // acc[cb][v]: channel 64 wv + 16 cb + 4 quad + v of column 16 cw + col.
    // Channel blocks pair up (0, 1), (2, 3) by one 16-lane row swap: an even
    // quad then holds channels 4 quad .. + 7 of the pair's first block (its
    // own and the next quad's), an odd quad channels 4 (quad - 1) .. + 7 of
    // the second, so every lane stores 16 contiguous bytes
    uint16_t* dst = A.part_o + chunk_partial_row(A, pko[cw], row_b, g, nslot, hh) * QSA_D + 64 * wv +
                    16 * (quad & 1) + 4 * (quad & 2);
#pragma unroll
    for (int cp = 0; cp < 4; cp += 2) {
      const auto lo = __builtin_amdgcn_permlane16_swap(pack_bf16x2(acc[cp][0], acc[cp][1]),
                                                       pack_bf16x2(acc[cp + 1][0], acc[cp + 1][1]), false, false);
      const auto hi = __builtin_amdgcn_permlane16_swap(pack_bf16x2(acc[cp][2], acc[cp][3]),
                                                       pack_bf16x2(acc[cp + 1][2], acc[cp + 1][3]), false, false);
      if (oko[cw]) *reinterpret_cast<u32x4_t*>(dst + 16 * cp) = u32x4_t{lo[0], hi[0], lo[1], hi[1]};
    }
  }
  if (mark) QM_PHASE(11);
}

// vmcnt(0) alone (expcnt and lgkmcnt at their maxima): the keys that went
// straight to LDS have landed before the barrier that hands them to the
// other waves
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__global__ __launch_bounds__(CA_NT, 4) void qsa_chunk_attend_kernel(ChunkAttnArgs A) {
  QM_PHASE_DECL
  QM_PHASE(0);
  const int x = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int col = lane & 15, quad = lane >> 4;
  const int il = col >> 3, hh = col & 7;
  const int nslot = A.topk + 1;
  const int gpb = A.ratio / 32;
  const int* ptab = A.page_table + (long)b * A.max_pages;
  const long row_b = (long)b * A.seq;                 // global index of the sequence's row 0
  const long head_stride = (long)A.page_size * QSA_D;
  const int e_w = 2 * wv + il;                        // this lane's entry within a group of 8

  __shared__ ChunkShared S;

  // A block's key pieces go straight to LDS (the wave's 4 of the 16 pieces of
  // each 32-token group, 1 KB each, lane l's 16 bytes at byte 16 l); the
  // wave's value pieces (channel blocks 4 wv .. 4 wv + 3 of each group) stay
  // in registers.
  bf16x8_t vr[2][4];   // set for the groups the block has
  // addressed through a buffer resource per group (a scalar base) and one
  // lane offset shared by every piece, the piece's offset scalar or immediate
  const int k_off = lane * 16 + wv * 1024, v_off = lane * 16 + wv * 4096;
  auto k_load = [&](int j, int page0, int page1) __attribute__((always_inline)) {
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      if (gi >= gpb) continue;
      const int rowg = (j * A.ratio + 32 * gi) % A.page_size;
      const long pbase = ((long)(gi ? page1 : page0) * A.hkv + g) * head_stride;
      const auto kr = dev_rsrc(A.k_pool + pbase + (rowg >> 4) * 8 * 512, 16 * 1024);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (__attribute__((address_space(3))) void*)&S.k[gi][wv + 4 * i][0],
                                                 16, k_off, 4096 * i, 0, 0);
    }
  };
  auto v_load = [&](int j, int page0, int page1) __attribute__((always_inline)) {
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      if (gi >= gpb) continue;
      const int rowg = (j * A.ratio + 32 * gi) % A.page_size;
      const long pbase = ((long)(gi ? page1 : page0) * A.hkv + g) * head_stride;
      const auto vrs = dev_rsrc(A.v_pool + pbase + (rowg >> 5) * 16 * 512, 16 * 1024);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        vr[gi][cb] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(vrs, v_off + 1024 * cb, 0, 0));
    }
  };
  // the chunk path scores with the query's bf16 part (hi) alone: the keys
  // are bf16 too, and the softmax of these 64-key blocks is far inside the
  // output tolerance either way, at half the query traffic and products
  bf16x8_t qhi[8];
  auto q_load = [&](unsigned pk) __attribute__((always_inline)) {
    const long row = row_b + (pk >> 16);
    const uint16_t* qh = A.q + q_index(row, A.hkv, 0, g * GQA + hh, 8 * quad);
#pragma unroll
    for (int sk = 0; sk < 8; ++sk) qhi[sk] = load_bf16x8(qh + Q_SK_STRIDE * sk);
  };
  auto pages_of = [&](int j, int& page0, int& page1) __attribute__((always_inline)) {
    page0 = ptab[min((j * A.ratio) / A.page_size, A.max_pages - 1)];
    page1 = ptab[min((j * A.ratio + (gpb > 1 ? 32 : 0)) / A.page_size, A.max_pages - 1)];
  };

  if (x < A.nwg_sel) {
    // ---- block j = x: the first 128 rows of its table row, its pages and
    // the position in one round trip; then its entries in groups of 8
    const int j = x;
    const uint16_t* trow = A.tab + ((long)b * A.max_blocks + j) * A.seq;
    const int ta = lane < A.seq ? trow[lane] : 0;
    const int tb = 64 + lane < A.seq ? trow[64 + lane] : 0;
    int page0, page1;
    pages_of(j, page0, page1);
    const int pos0 = A.positions[b];
    bool loaded = false, first = true;
    for (int c = 0; 128 * c < A.seq; ++c) {
      // rows 128 c + lane and 128 c + 64 + lane of the table row
      const int ra = 128 * c + lane, rb = ra + 64;
      const int tva = c == 0 ? ta : ra < A.seq ? trow[ra] : 0;
      const int tvb = c == 0 ? tb : rb < A.seq ? trow[rb] : 0;
      unsigned long long la = __ballot(tva != 0), lb = __ballot(tvb != 0);
      if ((la | lb) == 0ull) continue;
      const int nc = __popcll(la) + __popcll(lb);
      const unsigned ma = (static_cast<unsigned>(ra) << 16) | static_cast<unsigned>(tva - 1);
      const unsigned mb = (static_cast<unsigned>(rb) << 16) | static_cast<unsigned>(tvb - 1);
      bool fresh = false;
      if (!loaded) {
        // every wave is done with the keys of an earlier span (the barrier
        // between its last group's scores and outputs)
        k_load(j, page0, page1);
        v_load(j, page0, page1);
        loaded = fresh = true;
      }
      for (int g0 = 0; g0 < nc; g0 += 8) {
        // the group's entries: pko[cw] = entry 2 cw + il
        unsigned pko[4];
        next_group(la, lb, ma, mb, il, pko);
        const bool ok = g0 + e_w < nc;
        const unsigned pk = pick4(pko, wv);
        q_load(pk);
        if (fresh) {
          wait_loads();
          fresh = false;
        }
        __syncthreads();   // the block's keys are in LDS (and the previous group's weights read)
        if (first) QM_PHASE(3);
        if (g0 + 2 * wv < nc) chunk_scores(A, S, qhi, j, pk, ok, row_b, pos0, g, nslot, first);
        else chunk_no_scores(S);
        bool oko[4];
#pragma unroll
        for (int cw = 0; cw < 4; ++cw) oko[cw] = g0 + 2 * cw + il < nc;
        __syncthreads();
        chunk_outputs(A, S, vr, pko, oko, row_b, g, nslot, first);
        first = false;
      }
    }
  } else {
    // ---- the tail entries (keys ts..p) of rows tr0 .. tr0 + 7: block jt, then
    // block jt + 1 when the rows cross a block boundary
    const int tr0 = (x - A.nwg_sel) * CA_TAIL_ROWS;
    const int pos0 = A.positions[b];
    const int jt = (pos0 + tr0) / A.ratio;
    // entry e of the workgroup (row tr0 + e): its packed (row, tail, slot) and
    // whether its tail lies in block j
    auto tail_entry = [&](int e, int j, unsigned& pk) __attribute__((always_inline)) {
      const int r = tr0 + e, p = pos0 + r;
      pk = (static_cast<unsigned>(min(r, A.seq - 1)) << 16) | (1u << 9) | static_cast<unsigned>(A.topk);
      return r < A.seq && ((p + 1) / A.ratio) * A.ratio <= p && p / A.ratio == j;
    };
    int pa0, pa1, pb0, pb1;
    pages_of(jt, pa0, pa1);
    pages_of(jt + 1, pb0, pb1);
    unsigned pk;
    tail_entry(e_w, jt, pk);
    q_load(pk);
    for (int bi = 0; bi < 2; ++bi) {
      const int j = jt + bi;
      unsigned pko[4];
      bool oko[4];
#pragma unroll
      for (int cw = 0; cw < 4; ++cw) oko[cw] = tail_entry(2 * cw + il, j, pko[cw]);
      unsigned pk_j;
      const bool mine = tail_entry(e_w, j, pk_j);
      // whether any of the 8 rows has its tail in block j (every lane tests
      // them all, so the answer is uniform without an exchange)
      bool any = false;
#pragma unroll
      for (int e = 0; e < CA_TAIL_ROWS; ++e) {
        unsigned pe;
        any |= tail_entry(e, j, pe);
      }
      if (!any) continue;
      __syncthreads();   // every wave is done with the previous block's keys and weights
      k_load(j, bi ? pb0 : pa0, bi ? pb1 : pa1);
      v_load(j, bi ? pb0 : pa0, bi ? pb1 : pa1);
      wait_loads();
      __syncthreads();
      if (__builtin_amdgcn_ballot_w64(mine) != 0ull) chunk_scores(A, S, qhi, j, pk, mine, row_b, pos0, g, nslot);
      else chunk_no_scores(S);
      __syncthreads();
      chunk_outputs(A, S, vr, pko, oko, row_b, g, nslot);
    }
  }
  QM_PHASE(4);
  QM_PHASE_FLUSH();
}

// ---------------------------------------------------------------------------
// decode step: one launch per token
// ---------------------------------------------------------------------------
// qsa_decode_kernel, grid (G, kv head g, sequence b) of 256-thread workgroups,
// G at least the position's number of 32-token attention items. Workgroup x
// attends item x: spreading the key/value reads over one item per compute
// unit is what lets them run near the memory system's speed (a unit reading
// four items' 128 KB takes twice as long as four units reading 32 KB each).
// A workgroup:
//   0. issues its loads, every one of them unconditional and, but for the
//      rope row and a completed block's raw keys, independent of the position:
//      its 8 query heads, the token's key and value, the indexer query and
//      key, the norm weights, the page-table row, the first 128 block keys and
//      the group's generation word, so they share one round trip;
//   1. RMS-norms and ropes the indexer query and the pooled block key (sums of
//      squares in torch's order);
//   2. scores the eligible blocks and ranks them (redundantly in every
//      workgroup whose item is a selected block's: ~65 KB of L2-resident reads,
//      cheaper than a hand-off between workgroups);
//   3. issues its item's key/value loads (waves 0-1: the two 16-token key
//      tiles; wave w: value channels 64w..64w+63), then norms and ropes the 8
//      query heads and the key while they are in flight;
//   4. scores the item on bf16 MFMA (waves 0-1), shares the scores through LDS,
//      and every wave forms the softmax weights and its 64 output channels;
//      the current token's key/value come from LDS, not the pages;
//   5. writes the item's partial through to the device's point of coherence:
//      (max, sum) in float32, the output divided by the sum in bf16. The workgroup of item 0 also appends
//      the token's key/value to its page slot, and for kv head 0 writes the
//      per-sequence outputs (raw indexer key, pooled key);
//   6. raises its flag, and, when it holds one of the 64 (query head, 32
//      channels) slices of the group's output, waits for the flags of every
//      item of the group, merges that slice's partials and applies the gate.
// When the plan has fewer than 64 items (short contexts), the grid is widened
// to 64 workgroups per group so that every slice has its own merger (a
// workgroup merging several slices pays a round trip per slice): those past
// the position's items only merge, and raise their flag as soon as they have
// read the generation word; workgroup 0 then advances the word only after it
// has seen the flags of all 64, so that no workgroup reads the advanced word in
// the launch that advances it. Otherwise the attending workgroups merge the
// slices among themselves and only their flags are waited for.
// Every workgroup of a group must be resident at once for the waits to end.
// Workgroups are dispatched in order, so at most one group is ever partly
// dispatched; qm_qsa_decode refuses a group larger than the device's resident
// capacity for the kernel variant (occupancy x compute units, computed on the
// host), and callers route such plans to front + attend.
constexpr int DEC_WAVES = 4;
constexpr int DEC_NT = 64 * DEC_WAVES;
constexpr int DEC_MAX_BLOCKS = 2048;
constexpr int DEC_MAX_PAGES = 2048;
constexpr int DEC_MAX_TOPK = 256;
constexpr int DEC_MAX_ITEMS = 1024;   // workgroups per (sequence, kv head)
constexpr int DEC_MAX_RATIO = 64;     // raw keys of a completed block are held in registers
constexpr int DEC_GEN_STRIDE = 32;    // generation words 128 bytes apart, one cache line each
constexpr int DEC_SLICES = GQA * QSA_D / 32;   // output slices of a group: (query head, 32 channels)

template <typename T>
struct DecArgs {
  PrepArgs<T> P;
  uint16_t* part_o; float* part_ml;     // per group: [G][8][256] bf16 outputs / sum, [G][8] (max, sum)
  unsigned* gen;                        // per group: generation word, then a give-up counter
  unsigned* flags;                      // per group: G flags
  T* out;
  int* ids; int* n_sel; int2* items; float* iq_out;   // optional inspection outputs
  int splits, topk, max_items;
};

struct DecShared {
  unsigned long long key[DEC_MAX_BLOCKS];         // selection keys
  float4 dsc[128];                                // a round's per-block dot products (4 heads)
  float red[264];                                 // merge: partial sums and wave values
  int fault[DEC_WAVES];                           // the merge's waves whose wait gave up
  float iq[4 * IDX_D];                            // the roped indexer query rows
  float newkey[IDX_D];                            // the pooled key of the block this token completes
  alignas(16) uint16_t knb[QSA_D];                // the token's roped key and its value, bf16
  alignas(16) uint16_t vnb[QSA_D];
  alignas(16) uint16_t qb[16][QSA_D];             // MFMA B operand: rows 0..7 bf16 hi of the heads, 8..15 lo
  float chunk[DEC_MAX_RATIO / 16][IDX_D];
  int pages[DEC_MAX_PAGES];
  int sel[DEC_MAX_TOPK];
  alignas(16) int rscr[rank_scratch(DEC_MAX_TOPK)];
  alignas(16) float s[GQA][32];                   // the item's scores, head-major
};

// item -> (first token t0, visible rows [lo, hi)) of a query at position p
__device__ __forceinline__ void item_span(int it, int n_blk_items, int gpb, int ratio, int ts, int p, const int* sel,
                                          int& t0, int& lo, int& hi) {
  if (it < n_blk_items) {
    const int bs = sel[it / gpb] * ratio;
    if (ratio >= 32) { t0 = bs + (it % gpb) * 32; lo = 0; hi = 32; }
    else { t0 = bs & ~31; lo = bs - t0; hi = lo + ratio; }
  } else {
    t0 = (ts & ~31) + (it - n_blk_items) * 32; lo = max(ts - t0, 0); hi = min(p + 1 - t0, 32);
  }
}

// item_span with the item's selected block given (blk, for it < n_blk_items)
__device__ __forceinline__ void item_span_blk(int it, int n_blk_items, int gpb, int ratio, int ts, int p, int blk,
                                              int& t0, int& lo, int& hi) {
  if (it < n_blk_items) {
    const int bs = blk * ratio;
    if (ratio >= 32) { t0 = bs + (it % gpb) * 32; lo = 0; hi = 32; }
    else { t0 = bs & ~31; lo = bs - t0; hi = lo + ratio; }
  } else {
    t0 = (ts & ~31) + (it - n_blk_items) * 32; lo = max(ts - t0, 0); hi = min(p + 1 - t0, 32);
  }
}

// attention items of a query at position p (the selected blocks' 32-token
// groups, then the tail's)
struct ItemCount {
  int n_elig, n_sel, gpb, n_blk_items, ts, n_items;
  __host__ __device__ ItemCount(int p, int ratio, int topk, int max_blocks) {
    n_elig = min((p + 1) / ratio, max_blocks);
    n_sel = min(n_elig, topk);
    gpb = ratio >= 32 ? ratio / 32 : 1;
    n_blk_items = n_sel * gpb;
    ts = ((p + 1) / ratio) * ratio;
    const int n_tail = ts > p ? 0 : (p >> 5) - (ts >> 5) + 1;
    n_items = n_blk_items + n_tail;
  }
};

// flags of a group: one per workgroup that attends an item or holds a slice
__host__ __device__ inline int dec_flag_stride(int splits) { return splits > DEC_SLICES ? splits : DEC_SLICES; }

// Flags of the 128 items of round i0, polled by one wave (the caller's wave
// 0; its workgroup waits at a barrier): lane l polls items i0 + l and
// i0 + 64 + l, both loads issued together; items at or past n_wait count as
// raised. One polling wave per merging workgroup, not four: every poll of
// every merging workgroup reads the same few lines at the point of coherence,
// and fewer polls reach it sooner. False if the wait gave up.
__device__ __forceinline__ bool wait_item_flags(const unsigned* flags, int i0, int n_wait, unsigned target) {
  const int lane = threadIdx.x & 63;
  const int ia = i0 + lane, ib = ia + 64;
  const bool need_a = ia < n_wait, need_b = ib < n_wait;
  const unsigned* fa = flags + (need_a ? ia : 0);
  const unsigned* fb = flags + (need_b ? ib : 0);
  for (int k = 0; k < FLAG_SPIN_MAX; ++k) {
    const unsigned va = ld_flag(fa), vb = ld_flag(fb);
    const bool ok = (!need_a || (int)(va - target) >= 0) && (!need_b || (int)(vb - target) >= 0);
    if (__builtin_amdgcn_ballot_w64(!ok) == 0ull) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// Output slice sl = (query head h = sl / 8, channels 32 (sl % 8) ..+31) of
// group (b, g): out[d] = round(sum_i w_i o_i[d] / sum_i w_i) *
// round(sigmoid(gate[d])), w_i = exp(m_i - max m) l_i, over the n items (o_i
// is the item's output divided by its sum l_i). Thread (c = tid % 4, il =
// tid / 4) takes channels 8c .. 8c + 7 of the slice (one 16-byte load) of
// items il and il + 64 of each round of 128, so wave w merges items 16w ..
// 16w + 15 and 64 + 16w .. of a round; wave 0 waits for the round's flags
// (n_wait of them count), the workgroup meets at a barrier, and each wave
// loads its items' partials at once. Each thread keeps a running
// maximum, sum and 8 channel sums; the lanes of a chunk are added by DPP row
// rotations and lane swaps after scaling to the wave's maximum, and the four
// waves' (sums, maximum) meet in LDS. Workgroup 0 of the group advances the
// generation word (`word`, when given) once every wave has seen its flags.
// A wait that gives up counts itself in the group's give-up word and poisons
// the slice.
template <typename T>
__device__ void decode_combine_slice(const DecArgs<T>& D, DecShared& sh, int b, int g, int sl, int n, int n_wait,
                                     unsigned gen, bool overflow, float gate, unsigned* word,
                                     __amdgpu_buffer_rsrc_t ro, __amdgpu_buffer_rsrc_t rml) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c = tid & 3, il = tid >> 2;
  const int h = sl / 8, d0 = 32 * (sl % 8) + 8 * c;
  const int bg = b * D.P.hkv + g;
  const unsigned* flags = D.flags + (long)bg * dec_flag_stride(D.splits);
  float M = -INFINITY, L = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  bool ok = true;
  // the gate's sigmoid is formed while the first round's partials are in flight
  float gsig = 0.f;
  bool have_gate = false;
  const int n_rounds = max(n, n_wait);
  for (int i0 = 0; i0 < n_rounds; i0 += 128) {
    if (wv == 0) ok = ok & wait_item_flags(flags, i0, n_wait, gen + 1);
    __syncthreads();
    if (i0 >= n) continue;
    const int ia = i0 + il, ib = ia + 64;
    const int ca = min(ia, n - 1), cb = min(ib, n - 1);
    const u32x4_t oa = ld_dev_u32x4(ro, ((ca * GQA + h) * QSA_D + d0) * 2);
    const u32x4_t ob = ld_dev_u32x4(ro, ((cb * GQA + h) * QSA_D + d0) * 2);
    const float2 ma = ld_dev2(rml, ((ca * GQA + h) * 2) * 4);
    const float2 mb = ld_dev2(rml, ((cb * GQA + h) * 2) * 4);
    if (!have_gate) {
      gsig = Act<T>::round(sigmoid_f(gate));
      have_gate = true;
    }
    const float xa = ia < n ? ma.x : -INFINITY, xb = ib < n ? mb.x : -INFINITY;
    const float mn = fmaxf(M, fmaxf(xa, xb));
    const float f = M == -INFINITY ? 0.f : __expf(M - mn);
    const float wa = ia < n ? __expf(xa - mn) * ma.y : 0.f;
    const float wb = ib < n ? __expf(xb - mn) * mb.y : 0.f;
    L = L * f + wa + wb;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float va = __uint_as_float(e & 1 ? oa[e >> 1] & 0xffff0000u : oa[e >> 1] << 16);
      const float vb = __uint_as_float(e & 1 ? ob[e >> 1] & 0xffff0000u : ob[e >> 1] << 16);
      acc[e] = acc[e] * f + wa * va + wb * vb;
    }
    M = mn;
  }
  if (!have_gate) gsig = Act<T>::round(sigmoid_f(gate));
  // to the wave's maximum, then the sums over the wave's items (lanes of one c)
  const float Mw = wave_max(M);
  const float fw = M == -INFINITY ? 0.f : __expf(M - Mw);
  float v[9];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = acc[e] * fw;
  v[8] = L * fw;
#pragma unroll
  for (int e = 0; e < 9; ++e) {
    v[e] += dpp_f<0x124>(v[e]);     // row_ror:4
    v[e] += dpp_f<0x128>(v[e]);     // row_ror:8
    v[e] = xor32_sum(xor16_sum(v[e]));
  }
  float* red = sh.red;              // [wave][chunk][8 sums, L, M]
  if (lane < 4) {
#pragma unroll
    for (int e = 0; e < 9; ++e) red[(wv * 4 + lane) * 10 + e] = v[e];
    red[(wv * 4 + lane) * 10 + 9] = Mw;
  }
  if (lane == 0) {
    if (!ok) __hip_atomic_fetch_add(D.gen + (long)bg * DEC_GEN_STRIDE + 1, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    sh.fault[wv] = ok ? 0 : 1;
  }
  __syncthreads();
  QM_PHASE(9);
  if (word && tid == 0) st_flag(word, gen + 1);
  if (tid < 32) {
    const int cc = tid >> 3, e = tid & 7;
    float mw[DEC_WAVES], Mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) {
      mw[w] = red[(w * 4 + cc) * 10 + 9];
      Mx = fmaxf(Mx, mw[w]);
    }
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) {
      const float s = mw[w] == -INFINITY ? 0.f : __expf(mw[w] - Mx);
      num += red[(w * 4 + cc) * 10 + e] * s;
      den += red[(w * 4 + cc) * 10 + 8] * s;
    }
    const bool poison = overflow || (sh.fault[0] | sh.fault[1] | sh.fault[2] | sh.fault[3]) != 0;
    const int hq = D.P.hq, qh = g * GQA + h;
    const float y = Act<T>::round(num / den) * gsig;
    Act<T>::store(D.out, ((long)b * hq + qh) * QSA_D + 32 * (sl % 8) + tid, poison ? __builtin_nanf("") : y);
  }
  __syncthreads();
}

// Workgroup `item` < DEC_SLICES of group (b, g): merge output slices item,
// item + step, ... once the flags of the n_att attending workgroups have
// reached gen + 1 (workgroup 0 of a widened grid waits for all 64 slice
// holders' flags, then advances the generation word). A wait that gives up
// counts itself in the group's give-up word and the slices this workgroup
// merges become NaN (never a merge of missing partials); so do all slices
// when the position has more items than the launch has workgroups
// (`overflow`). qm_qsa_decode_check reads and resets both counters.
template <bool WIDE, typename T>
__device__ __forceinline__ void decode_merge(const DecArgs<T>& D, DecShared& sh, int b, int g, int item, int n_att,
                                             unsigned gen, bool overflow) {
  const int tid = threadIdx.x;
  const int bg = b * D.P.hkv + g;
  const long gbase = (long)bg * D.splits;
  const __amdgpu_buffer_rsrc_t ro = dev_rsrc(D.part_o + gbase * GQA * QSA_D, (long)D.splits * GQA * QSA_D * 2);
  const __amdgpu_buffer_rsrc_t rml = dev_rsrc(D.part_ml + gbase * GQA * 2, (long)D.splits * GQA * 2 * 4);
  const int n_wait = WIDE && item == 0 ? DEC_SLICES : n_att;
  const int step = WIDE ? DEC_SLICES : n_att;
  const int hq = D.P.hq;
  auto gate_of = [&](int sl) {
    return Act<T>::load(D.P.qg, ((long)b * hq + g * GQA + sl / 8) * (2 * QSA_D) + QSA_D + 32 * (sl % 8) + (tid & 31));
  };
  // the first slice's gate is loaded before the wait
  const float gate0 = gate_of(item);
  unsigned* word = item == 0 ? D.gen + (long)bg * DEC_GEN_STRIDE : nullptr;
  for (int sl = item; sl < DEC_SLICES; sl += step) {
    decode_combine_slice(D, sh, b, g, sl, n_att, n_wait, gen, overflow, sl == item ? gate0 : gate_of(sl),
                         sl == item ? word : nullptr, ro, rml);
  }
}

// The arguments the first loads need come first, as plain scalars: the library
// is built with kernel-argument preloading, so these 14 dwords are in scalar
// registers at wave start and the position, the indexer query and its norm
// weight and the block keys are requested at once, then the rope rows as soon
// as the position is in; the rest of the arguments (D) arrive by the kernel's
// own scalar loads while those are in flight. dims0 = max_blocks | rope << 16
// | idx_heads << 24 | may_score << 28, where may_score says the launch's
// positions may need scoring (more items than the top-k blocks hold), so the
// first 128 block keys are prefetched whatever the position; dims1 =
// log2(ratio) | topk << 8.
template <typename T, bool WIDE>
__global__ __launch_bounds__(DEC_NT) void qsa_decode_kernel(const int* positions0, const T* iq0,
                                                            const float* iq_norm0, const float* bk0,
                                                            const float* cos0, const float* sin0, unsigned dims0,
                                                            unsigned dims1, DecArgs<T> D) {
  __shared__ DecShared sh;
  QM_PHASE_DECL
  const PrepArgs<T>& A = D.P;
  const int item = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int col = lane & 15, quad = lane >> 4;
  const int e128 = tid & 127, hh = tid >> 7;
  const int max_blocks = dims0 & 0xffff, rope = (dims0 >> 16) & 0xff, idx_heads = (dims0 >> 24) & 0xf;
  const bool may_score = (dims0 >> 28) & 1;
  const int ratio_log2 = dims1 & 0xff, ratio = 1 << ratio_log2, topk = dims1 >> 8;

  // ---- 0. the loads. Wave w takes indexer query head w and attention query
  // heads 2w, 2w + 1 (wave 0 also the key), each row as elements lane + 64 k.
  // Every load is unconditional, indices clamped into range, so the waits on
  // them stay exact instead of draining the memory counter. First the ones
  // the scalar arguments address: the position (a vector load, issued first:
  // a scalar load would be issued after the scalar loads of D and waited for
  // with them), the indexer query and its norm weight, the first 128 block
  // keys, then the rope rows of this token's position and of the start of the
  // block it completes.
  QM_PHASE(0);
  const int p = __builtin_amdgcn_readfirstlane(
      (int)__builtin_amdgcn_raw_buffer_load_b32(dev_rsrc(positions0 + b, 4), 0, 0, 0));
  const int n_iq = idx_heads * IDX_D;
  float iqx[2], w_iq[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) iqx[k] = Act<T>::load(iq0, (long)b * n_iq + min(wv * IDX_D + lane + 64 * k, n_iq - 1));
#pragma unroll
  for (int k = 0; k < 2; ++k) w_iq[k] = iq_norm0[lane + 64 * k];
  const float* bk = bk0 + (long)b * max_blocks * IDX_D;
  float kp[score_pre<DEC_NT>()][8];
  prefetch_block_keys_raw<DEC_NT>(kp, bk, max_blocks, may_score);
  // every block-key load issued before the wait for the position
  __builtin_amdgcn_sched_barrier(0);
  const int j_new = ((p + 1) & (ratio - 1)) == 0 ? p >> ratio_log2 : -1;
  float cs[2], sn[2], cs0[2], sn0[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int ec = min(lane + 64 * k, rope - 1);
    cs[k] = cos0[(long)p * rope + ec];
    sn[k] = sin0[(long)p * rope + ec];
    cs0[k] = cos0[(long)max(j_new, 0) * ratio * rope + ec];
    sn0[k] = sin0[(long)max(j_new, 0) * ratio * rope + ec];
  }
  // nothing addressed through D moves above this point: its scalar loads'
  // waits would hold up the rope rows
  __builtin_amdgcn_sched_barrier(0);
  // then the loads addressed through D: the page-table row (for after the
  // selection), the generation word, the token's inputs and norm weights
  int pg[DEC_MAX_PAGES / DEC_NT];
#pragma unroll
  for (int k = 0; k < DEC_MAX_PAGES / DEC_NT; ++k)
    pg[k] = A.page_table[(long)b * A.max_pages + min(tid + DEC_NT * k, A.max_pages - 1)];
  const int bg = b * A.hkv + g;
  const unsigned gen = ld_flag(D.gen + (long)bg * DEC_GEN_STRIDE);
  const float ikv = Act<T>::load(A.ik, (long)b * IDX_D + e128);
  float qx[2][4], kx[4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k)
      qx[j][k] = Act<T>::load(A.qg, ((long)b * A.hq + g * GQA + 2 * wv + j) * (2 * QSA_D) + lane + 64 * k);
#pragma unroll
  for (int k = 0; k < 4; ++k) kx[k] = Act<T>::load(A.k_new, (long)bg * QSA_D + lane + 64 * k);
  const float vx = Act<T>::load(A.v_new, (long)bg * QSA_D + tid);
  float w_q[4], w_k[4], w_ik[2];
#pragma unroll
  for (int k = 0; k < 4; ++k) { w_q[k] = A.q_norm[lane + 64 * k]; w_k[k] = A.k_norm[lane + 64 * k]; }
#pragma unroll
  for (int k = 0; k < 2; ++k) w_ik[k] = A.ik_norm[lane + 64 * k];

  const ItemCount ic(p, ratio, topk, max_blocks);
  const int n_elig = ic.n_elig, n_items = ic.n_items;
  const bool scoring = n_elig > topk;
  // raw keys of the block this token completes: thread (e128, hh) takes the
  // 16-row chunks hh and hh + 2; the token's own row is ik (not yet stored)
  float rk[2][16];
  if (j_new >= 0) {
    const T* raw = A.raw_keys + ((long)b * A.max_ctx + (long)j_new * ratio) * IDX_D + e128;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 16 * (hh + 2 * c) + i;
        const float v = Act<T>::load(raw, (long)min(r, ratio - 1) * IDX_D);
        rk[c][i] = r >= ratio ? 0.f : j_new * ratio + r == p ? ikv : v;
      }
  }

  // A position with more items than the launch has workgroups (a plan sized
  // for smaller positions) cannot be attended: its output is poisoned and
  // workgroup 0 counts it in the group's word 2. A workgroup past the
  // position's items only merges: the waits of this launch cover only the
  // first n_att flags.
  const bool overflow = n_items > D.splits;
  const int n_att = min(n_items, D.splits);
  if (overflow && item == 0 && tid == 0)
    __hip_atomic_fetch_add(D.gen + (long)bg * DEC_GEN_STRIDE + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (item >= n_att) {
    if constexpr (WIDE) {
      // a slice holder past the items: flag raised once the word is read
      if (item < DEC_SLICES) {
        if (tid == 0) raise_flag(D.flags + (long)bg * dec_flag_stride(D.splits) + item, gen + 1);
        decode_merge<WIDE>(D, sh, b, g, item, n_att, gen, overflow);
      }
    }
    QM_PHASE_FLUSH();
    return;
  }
  const bool blk_item = item < ic.n_blk_items;

  // ---- 1. the indexer query (wave w: head w), and the pooled key of a block
  // this token completes: y = round_T(x * rinv * w), then rope
  auto nrm = [&](float xv, float ri, float w) { return Act<T>::round(mul_rn(mul_rn(xv, ri), w)); };
  if (wv < idx_heads) {
    const float ri = wave_rinv<2>(iqx, A.eps);
    QM_PHASE(1);
    float y[2] = {nrm(iqx[0], ri, w_iq[0]), nrm(iqx[1], ri, w_iq[1])};
    wave_rope<2>(y, rope, cs, sn);
    sh.iq[wv * IDX_D + lane] = y[0];
    sh.iq[wv * IDX_D + 64 + lane] = y[1];
  } else {
    sh.iq[wv * IDX_D + lane] = 0.f;
    sh.iq[wv * IDX_D + 64 + lane] = 0.f;
  }
  if (j_new >= 0) {
    // block mean: the 16-row chunk sums in order, then divided by the count
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int ch = hh + 2 * c;
      if (16 * ch < ratio) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (16 * ch + i < ratio) acc = add_rn(acc, rk[c][i]);
        sh.chunk[ch][e128] = acc;
      }
    }
    __syncthreads();
    if (wv == 0) {
      float x[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        float total = sh.chunk[0][lane + 64 * k];
        for (int ch = 1; 16 * ch < ratio; ++ch) total = add_rn(total, sh.chunk[ch][lane + 64 * k]);
        x[k] = Act<T>::round(div_rn(total, (float)ratio));
      }
      const float ri = wave_rinv<2>(x, A.eps);
      float y[2] = {nrm(x[0], ri, w_ik[0]), nrm(x[1], ri, w_ik[1])};
      wave_rope<2>(y, rope, cs0, sn0);
      sh.newkey[lane] = y[0];
      sh.newkey[64 + lane] = y[1];
    }
  }
  // the token's value and the page-table row, for after the selection (the
  // rope above has waited for the loads issued before the rope rows)
  sh.vnb[tid] = f32_to_bf16(vx);
#pragma unroll
  for (int k = 0; k < DEC_MAX_PAGES / DEC_NT; ++k) sh.pages[tid + DEC_NT * k] = pg[k];
  __syncthreads();

  // ---- 2. block scores and top-k (ties to the lower index); the item of a
  // tail workgroup does not depend on them
  // The item's block is known without reading sel back when the selection
  // is select128's (it returns the block) or there is none (block i is the
  // i-th); after the counting ranks of rank_topk, sel is read behind a barrier.
  QM_PHASE(2);
  int blk = blk_item && !scoring ? item / ic.gpb : -1;
  if (scoring && (blk_item || item == 0)) {
    if (!score_block_rounds<DEC_NT, score_pre<DEC_NT>()>(sh.iq, sh.newkey, bk, n_elig, j_new, idx_heads, sh.key,
                                                         sh.dsc, kp, topk, sh.sel, blk_item ? item / ic.gpb : -1,
                                                         &blk)) {
      __syncthreads();
      QM_PHASE(3);
      rank_topk<DEC_NT, DEC_MAX_TOPK>(sh.key, n_elig, topk, sh.sel, sh.rscr);
      __syncthreads();
      blk = blk_item ? sh.sel[item / ic.gpb] : -1;
    }
  } else if (!scoring) {
    for (int i = tid; i < n_elig; i += DEC_NT) sh.sel[i] = i;
  }

  // ---- 3. the item's keys/values in flight while the query heads and key are normed
  QM_PHASE(4);
  int t0, lo, hi;
  item_span_blk(item, ic.n_blk_items, ic.gpb, ratio, ic.ts, p, blk, t0, lo, hi);
  const int page = sh.pages[t0 / A.page_size], row0 = t0 % A.page_size;
  const long pbase = ((long)page * A.hkv + g) * A.page_size * QSA_D;
  // Every earlier load has landed by now (the selection used them): saying so
  // lets the compiler issue the value and key loads back to back, instead of
  // waiting on the first of them for a register an earlier load might still
  // be writing.
  __builtin_amdgcn_s_waitcnt(0);
  bf16x8_t kf[8], vf[4];
  {
    const uint16_t* vt = A.v_pool + pbase + ((row0 >> 5) * 16 + 4 * wv) * 512 + lane * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) vf[i] = load_bf16x8(vt + i * 512);
  }
  if (wv < 2) {
    const uint16_t* kt = A.k_pool + pbase + ((row0 >> 4) + wv) * 8 * 512 + lane * 8;
#pragma unroll
    for (int sk = 0; sk < 8; ++sk) kf[sk] = load_bf16x8(kt + sk * 512);
  }
  const bool cur = p >= t0 && p < t0 + 32;          // the item holds the current token
  const int rcur = p - t0;
  // wave w: query heads 2w, 2w + 1 (and, in the workgroups that use it, wave 0
  // the key), normed and roped; the attention MFMA takes q as bf16 hi + lo
  // (~16 mantissa bits)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int h = 2 * wv + j;
    const float ri = wave_rinv_fast(qx[j], A.eps);
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = nrm(qx[j][k], ri, w_q[k]);
    wave_rope<4>(y, rope, cs, sn);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t qhi = f32_to_bf16(y[k]);
      sh.qb[h][lane + 64 * k] = qhi;
      sh.qb[GQA + h][lane + 64 * k] = f32_to_bf16(y[k] - bf16_to_f32(qhi));
    }
  }
  // the token's roped key, in the bits appended to the cache: before the
  // scores in the workgroup whose item holds the token; item 0, which appends
  // it, forms it after raising its flag (below) when it does not hold it
  auto key_bits = [&]() {
    const float ri = wave_rinv<4>(kx, A.eps);
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = nrm(kx[k], ri, w_k[k]);
    wave_rope<4>(y, rope, cs, sn);
#pragma unroll
    for (int k = 0; k < 4; ++k) sh.knb[lane + 64 * k] = f32_to_bf16(y[k]);
  };
  if (wv == 0 && cur) key_bits();
  QM_PHASE(5);
  __syncthreads();

  // ---- 4. scores of the item's two 16-token tiles (waves 0, 1)
  if (wv < 2) {
    if (cur && (rcur >> 4) == wv) {
      // the current token's key replaces whole 8-channel vectors of one lane
      const bool krow = col == (rcur & 15);
#pragma unroll
      for (int sk = 0; sk < 8; ++sk) {
        const bf16x8_t kv = *reinterpret_cast<const bf16x8_t*>(&sh.knb[32 * sk + 8 * quad]);
        kf[sk] = krow ? kv : kf[sk];
      }
    }
    // S^T = K Q^T: columns 0..7 take q hi, 8..15 q lo; lane col then adds its
    // partner column col ^ 8 (DPP row rotate by 8) for the full-precision score
    f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sk = 0; sk < 8; ++sk) {
      const bf16x8_t qf = *reinterpret_cast<const bf16x8_t*>(&sh.qb[col][32 * sk + 8 * quad]);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[sk], qf, c, 0, 0, 0);
    }
    float4 sv;
    float* svp = reinterpret_cast<float*>(&sv);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int tok = 16 * wv + 4 * quad + v;
      const float full = c[v] + dpp_f<0x128>(c[v]);
      svp[v] = (tok >= lo && tok < hi) ? full * (1.0f / 16.0f) : -INFINITY;
    }
    if (col < GQA) *reinterpret_cast<float4*>(&sh.s[col][16 * wv + 4 * quad]) = sv;
  }
  QM_PHASE(6);
  __syncthreads();
  // softmax weights: lane (col, quad) takes tokens 16t + 4quad + v of head col
  // (t = 0, 1), the k order the PV MFMA's B operand wants
  const int hcol = col & 7;
  const float4 s0 = *reinterpret_cast<const float4*>(&sh.s[hcol][4 * quad]);
  const float4 s1 = *reinterpret_cast<const float4*>(&sh.s[hcol][16 + 4 * quad]);
  const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < 8; ++i) mx = fmaxf(mx, sv[i]);
  mx = xor32_max(xor16_max(mx));
  float pv[8];
  float lsum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    pv[i] = __expf(sv[i] - mx);
    lsum += pv[i];
  }
  u32x4_t pu;
#pragma unroll
  for (int i = 0; i < 4; ++i) pu[i] = col < GQA ? pack_bf16x2(pv[2 * i], pv[2 * i + 1]) : 0u;
  const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, pu);
  lsum = xor32_sum(xor16_sum(lsum));
  QM_PHASE(12);
  if (cur) {
    // the current token's value: one element (column kappa) of the lanes whose
    // quad holds that column
    const int kappa = v_slot(rcur);
    const int dw = (kappa & 7) >> 1, sh16 = 16 * (kappa & 1);
    const bool vcol = quad == (kappa >> 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const unsigned val = sh.vnb[16 * (4 * wv + i) + col];
      u32x4_t u = __builtin_bit_cast(u32x4_t, vf[i]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (vcol && j == dw) u[j] = (u[j] & ~(0xffffu << sh16)) | (val << sh16);
      vf[i] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  // O^T[d][head] = V^T[d][tok] P^T[tok][head] for this wave's 64 channels,
  // written through to the point of coherence (read by other workgroups)
  const long gbase = (long)bg * D.splits;
  const __amdgpu_buffer_rsrc_t ro = dev_rsrc(D.part_o + gbase * GQA * QSA_D, (long)D.splits * GQA * QSA_D * 2);
  const __amdgpu_buffer_rsrc_t rml = dev_rsrc(D.part_ml + gbase * GQA * 2, (long)D.splits * GQA * 2 * 4);
  const float linv = 1.0f / lsum;
  // all four products before any store: a store ahead of a later load's wait
  // would be waited for too (the counter covers both, in order)
  f32x4_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[i], pf, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
  if (col < GQA) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const unsigned lo = pack_bf16x2(o[i][0] * linv, o[i][1] * linv);
      const unsigned hi = pack_bf16x2(o[i][2] * linv, o[i][3] * linv);
      st_dev_u32x2(ro, ((item * GQA + hcol) * QSA_D + 16 * (4 * wv + i) + 4 * quad) * 2, lo, hi);
    }
  }
  if (wv == 0 && quad == 0 && col < GQA) st_dev2(rml, ((item * GQA + col) * 2) * 4, make_float2(mx, lsum));
  QM_PHASE(7);

  // ---- 5. arrive: the partial's stores acknowledged, then the flag; the
  // workgroups holding output slices then wait for every item of the group
  // and merge their slices (6)
  wait_all_memory();
  __syncthreads();
  QM_PHASE(8);
  if (tid == 0) post_flag(D.flags + (long)bg * dec_flag_stride(D.splits) + item, gen + 1);

  // the stores that outlive this step, after the flag (no merge waits for
  // them; the launch's end does): the token's key/value into its page slot
  // (item 0 of each kv head), and per sequence (item 0 of kv head 0) its raw
  // indexer key, the pooled key of a completed block and the optional
  // inspection outputs
  if (item == 0) {
    if (!cur) {
      if (wv == 0) key_bits();
      __syncthreads();
    }
    const int pg_cur = sh.pages[p / A.page_size], prow = p % A.page_size;
    const long cbase = ((long)pg_cur * A.hkv + g) * A.page_size * QSA_D;
    A.k_pool[cbase + k_page_index(prow, tid)] = sh.knb[tid];
    A.v_pool[cbase + v_page_index(prow, tid)] = sh.vnb[tid];
    if (g == 0) {
      if (tid < IDX_D) {
        Act<T>::store(A.raw_keys, ((long)b * A.max_ctx + p) * IDX_D + tid, ikv);
        if (j_new >= 0) A.block_keys[((long)b * A.max_blocks + j_new) * IDX_D + bk_index(tid)] = sh.newkey[tid];
      }
      if (D.iq_out)
        for (int i = tid; i < A.idx_heads * IDX_D; i += DEC_NT) D.iq_out[(long)b * A.idx_heads * IDX_D + i] = sh.iq[i];
      if (D.items) {
        int2* items = D.items + (long)b * D.max_items;
        for (int it = tid; it < n_items; it += DEC_NT) {
          int u0, ulo, uhi;
          item_span(it, ic.n_blk_items, ic.gpb, ratio, ic.ts, p, sh.sel, u0, ulo, uhi);
          items[1 + it] = make_item(sh.pages[u0 / A.page_size] * A.page_size + u0 % A.page_size, ulo, uhi);
        }
        if (tid == 0) items[0] = make_int2(n_items, 0);
      }
      if (D.ids) {
        for (int i = tid; i < ic.n_sel; i += DEC_NT) D.ids[(long)b * topk + i] = sh.sel[i];
        if (tid == 0) D.n_sel[b] = ic.n_sel;
      }
    }
  }

  // ---- 6. the merge of this workgroup's output slices
  if (item < DEC_SLICES) decode_merge<WIDE>(D, sh, b, g, item, n_att, gen, overflow);
  QM_PHASE(10);
  QM_PHASE_FLUSH();
}

// Hides a value's origin from the optimiser, so that its conversion is not
// moved up to where it is loaded (which would wait for the load there).
__device__ __forceinline__ void opaque(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void opaque(bf16_t& v) {
  unsigned u = v.bits;
  asm volatile("" : "+v"(u));
  v.bits = static_cast<uint16_t>(u);
}

// ---------------------------------------------------------------------------
// Short-context decode: selection off and at most SL_MAX_TOK keys, with no
// hand-off between workgroups. Workgroup x < 64 of (kv head g, sequence b)
// owns output slice x = (query head h = x / 8, channels 32 (x % 8) .. + 31): it
// scores every key 0..p against query head h (K tiles on bf16 MFMA, the query
// as its hi and lo columns), takes the softmax over them in LDS, and
// multiplies the weights by its 32 value channels (two PV MFMAs per 32-key
// group), so neither partials nor flags cross workgroups. Sixteen waves: wave
// w holds 16-key tiles w and w + 16 and 32-key group w, all requested as soon
// as the page-table row is in, so the keys and values cost one round trip.
// Each workgroup reads every key of its kv head (576 bytes per key with its
// value channels, from L2 after the first), which is why the path stops at
// SL_MAX_TOK keys. Workgroup 0 of each kv head also appends the token's key and
// value; workgroup 64 of kv head 0 stores the raw indexer key, pools the block
// the token completes and writes the optional inspection outputs. The
// arithmetic is the long-context kernel's (its scores, the bf16 softmax
// weights of the PV product, fp32 sums), with one softmax over all keys
// instead of a merge of per-item softmaxes.
constexpr int SL_MAX_TOK = 512;
// Plans up to this many 32-key items take it: each of its workgroups reads
// every key (the long-context kernel's fixed cost is reached near 448 keys)
constexpr int SL_FAST_ITEMS = 10;
constexpr int SL_MAX_PAGES = SL_MAX_TOK / 32;   // pages hold at least 32 rows
constexpr int SL_WAVES = 16;
constexpr int SL_NT = 64 * SL_WAVES;

struct SliceShared {
  alignas(16) uint16_t qb[2][QSA_D];            // query head h: bf16 hi and lo
  alignas(16) uint16_t knb[QSA_D];              // the token's roped key, bf16
  alignas(16) uint16_t vnb[QSA_D];              // the token's value, bf16
  float s[SL_MAX_TOK];                          // scores, then softmax weights
  float red[SL_WAVES][32];                      // the waves' output sums
  float wred[SL_WAVES];                         // the waves' score maxima
  float wsum[SL_WAVES];                         // the waves' weight sums
  int pages[SL_MAX_PAGES];
  float chunk[DEC_MAX_RATIO / 16][IDX_D];       // side workgroup: 16-row sums
};

// The sequence's side work (threads 0..255 of workgroup 64, kv head 0).
template <typename T>
__device__ void slices_side_work(const DecArgs<T>& D, SliceShared& sh, int b, int p) {
  const PrepArgs<T>& A = D.P;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int e128 = tid & 127, hh = tid >> 7;
  const bool act = tid < DEC_NT;
  const int rope = A.rope, ratio = A.ratio, topk = D.topk;
  const int j_new = (p + 1) % ratio == 0 ? p / ratio : -1;
  const float ikv = Act<T>::load(A.ik, (long)b * IDX_D + e128);
  auto nrm = [&](float xv, float ri, float w) { return Act<T>::round(mul_rn(mul_rn(xv, ri), w)); };
  if (tid < IDX_D) Act<T>::store(A.raw_keys, ((long)b * A.max_ctx + p) * IDX_D + tid, ikv);
  if (j_new >= 0) {
    // the block's mean (16-row chunk sums in order, then divided by the count),
    // cast, normed and roped at the block's first position; the token's own row
    // is ik (its store above may not be visible to these loads)
    if (act) {
      const T* raw = A.raw_keys + ((long)b * A.max_ctx + (long)j_new * ratio) * IDX_D + e128;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int ch = hh + 2 * c;
        if (16 * ch < ratio) {
          float acc = 0.f;
          for (int i = 0; i < 16 && 16 * ch + i < ratio; ++i) {
            const int r = 16 * ch + i;
            acc = add_rn(acc, j_new * ratio + r == p ? ikv : Act<T>::load(raw, (long)r * IDX_D));
          }
          sh.chunk[ch][e128] = acc;
        }
      }
    }
    __syncthreads();
    if (wv == 0) {
      float x[2], cs0[2], sn0[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        float total = sh.chunk[0][lane + 64 * k];
        for (int ch = 1; 16 * ch < ratio; ++ch) total = add_rn(total, sh.chunk[ch][lane + 64 * k]);
        x[k] = Act<T>::round(div_rn(total, (float)ratio));
        const int ec = min(lane + 64 * k, rope - 1);
        cs0[k] = A.cos[(long)j_new * ratio * rope + ec];
        sn0[k] = A.sin[(long)j_new * ratio * rope + ec];
      }
      const float ri = wave_rinv<2>(x, A.eps);
      float y[2] = {nrm(x[0], ri, A.ik_norm[lane]), nrm(x[1], ri, A.ik_norm[lane + 64])};
      wave_rope<2>(y, rope, cs0, sn0);
#pragma unroll
      for (int k = 0; k < 2; ++k)
        A.block_keys[((long)b * A.max_blocks + j_new) * IDX_D + bk_index(lane + 64 * k)] = y[k];
    }
  }
  if (D.iq_out && wv < A.idx_heads) {
    const int n_iq = A.idx_heads * IDX_D;
    float x[2], cs[2], sn[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      x[k] = Act<T>::load(A.iq, (long)b * n_iq + wv * IDX_D + lane + 64 * k);
      const int ec = min(lane + 64 * k, rope - 1);
      cs[k] = A.cos[(long)p * rope + ec];
      sn[k] = A.sin[(long)p * rope + ec];
    }
    const float ri = wave_rinv<2>(x, A.eps);
    float y[2] = {nrm(x[0], ri, A.iq_norm[lane]), nrm(x[1], ri, A.iq_norm[lane + 64])};
    wave_rope<2>(y, rope, cs, sn);
#pragma unroll
    for (int k = 0; k < 2; ++k) D.iq_out[(long)b * n_iq + wv * IDX_D + lane + 64 * k] = y[k];
  }
  const ItemCount ic(p, ratio, topk, A.max_blocks);
  if (D.ids) {
    for (int i = tid; i < ic.n_sel; i += SL_NT) D.ids[(long)b * topk + i] = i;
    if (tid == 0) D.n_sel[b] = ic.n_sel;
  }
  if (D.items) {
    int2* items = D.items + (long)b * D.max_items;
    for (int it = tid; it < ic.n_items; it += SL_NT) {
      int u0, ulo, uhi;
      item_span_blk(it, ic.n_blk_items, ic.gpb, ratio, ic.ts, p, it / ic.gpb, u0, ulo, uhi);
      const int pg = A.page_table[(long)b * A.max_pages + min(u0 / A.page_size, A.max_pages - 1)];
      items[1 + it] = make_item(pg * A.page_size + u0 % A.page_size, ulo, uhi);
    }
    if (tid == 0) items[0] = make_int2(ic.n_items, 0);
  }
}

template <typename T>
__global__ __launch_bounds__(SL_NT) void qsa_decode_slices_kernel(DecArgs<T> D) {
  __shared__ SliceShared sh;
  QM_PHASE_DECL
  QM_PHASE(0);
  const PrepArgs<T>& A = D.P;
  const int x = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int col = lane & 15, quad = lane >> 4;
  const int p = A.positions[b];
  if (x == DEC_SLICES) {
    // the side work belongs to the sequence, not to a kv head
    if (g == 0 && p + 1 <= SL_MAX_TOK) slices_side_work<T>(D, sh, b, p);
    QM_PHASE(8);
    QM_PHASE_FLUSH();
    return;
  }
  const int h = x >> 3, cb = x & 7, qh = g * GQA + h;
  const int hq = A.hq, rope = A.rope;
  const int bg = b * A.hkv + g;
  T* out = D.out + ((long)b * hq + qh) * QSA_D + 32 * cb;
  if (p + 1 > SL_MAX_TOK) {
    // a position past the short range (a plan sized for smaller positions)
    // cannot be attended: its output is poisoned and counted in word 2
    if (x == 0 && tid == 0)
      __hip_atomic_fetch_add(D.gen + (long)bg * DEC_GEN_STRIDE + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 32) Act<T>::store(out, tid, __builtin_nanf(""));
    return;
  }

  // ---- loads, every one unconditional (indices clamped) and none converted
  // where it is loaded, so that no wait comes before the last is issued: the
  // page-table row first (the key and value loads need it), the query head
  // (wave 0) or the token's key (the other waves; wave 1 uses it) with their
  // norm weights, the token's value, the gate of the slice's channels, then
  // the rope row once the position is in
  const int pgv = A.page_table[(long)b * A.max_pages + min(tid & (SL_MAX_PAGES - 1), A.max_pages - 1)];
  T xt[4], vt_raw, gt_raw;
  float wr[4], cs[2], sn[2];
  {
    const T* src = wv == 0 ? A.qg + ((long)b * hq + qh) * (2 * QSA_D) : A.k_new + (long)bg * QSA_D;
    const float* wsrc = wv == 0 ? A.q_norm : A.k_norm;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      xt[k] = src[lane + 64 * k];
      wr[k] = wsrc[lane + 64 * k];
    }
  }
  vt_raw = A.v_new[(long)bg * QSA_D + (tid & (QSA_D - 1))];
  gt_raw = A.qg[((long)b * hq + qh) * (2 * QSA_D) + QSA_D + 32 * cb + (tid & 31)];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int ec = min(lane + 64 * k, rope - 1);
    cs[k] = A.cos[(long)p * rope + ec];
    sn[k] = A.sin[(long)p * rope + ec];
  }
  if (tid < SL_MAX_PAGES) sh.pages[tid] = pgv;
  __syncthreads();                        // the page-table row in LDS
  QM_PHASE(1);

  // ---- the wave's keys and values, requested now so that they travel while
  // the query and key are normed: 16-key tiles wv and wv + 16, 32-key group wv
  // (a wave past the keys loads nothing; the branches are uniform per wave)
  const int n_tok = p + 1, n_tiles = (n_tok + 15) >> 4, n_grp = (n_tok + 31) >> 5;
  const long head_base = (long)g * A.page_size * QSA_D;
  const long page_stride = (long)A.hkv * A.page_size * QSA_D;
  bf16x8_t kf[2][8], vf[2];              // set only where used
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (wv + SL_WAVES * i < n_tiles) {
      const int r16 = 16 * (wv + SL_WAVES * i);
      const uint16_t* kt = A.k_pool + sh.pages[r16 / A.page_size] * page_stride + head_base +
                           ((r16 % A.page_size) >> 4) * 8 * 512 + lane * 8;
#pragma unroll
      for (int sk = 0; sk < 8; ++sk) kf[i][sk] = load_bf16x8(kt + sk * 512);
    }
  }
  if (wv < n_grp) {
    const int r32 = 32 * wv;
    const uint16_t* vt = A.v_pool + sh.pages[r32 / A.page_size] * page_stride + head_base +
                         (((r32 % A.page_size) >> 5) * 16 + 2 * cb) * 512 + lane * 8;
#pragma unroll
    for (int j = 0; j < 2; ++j) vf[j] = load_bf16x8(vt + j * 512);
  }
  QM_PHASE(2);

  auto nrm = [&](float xv, float ri, float w) { return Act<T>::round(mul_rn(mul_rn(xv, ri), w)); };
  float xr[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    opaque(xt[k]);
    xr[k] = Act<T>::load(&xt[k], 0);
  }
  if (wv == 0) {
    // the query head: fused sum of squares and the hardware reciprocal square
    // root (as the long-context kernel), then bf16 hi and lo
    const float ri = wave_rinv_fast(xr, A.eps);
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = nrm(xr[k], ri, wr[k]);
    wave_rope<4>(y, rope, cs, sn);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t qhi = f32_to_bf16(y[k]);
      sh.qb[0][lane + 64 * k] = qhi;
      sh.qb[1][lane + 64 * k] = f32_to_bf16(y[k] - bf16_to_f32(qhi));
    }
  } else if (wv == 1) {
    // the token's key, in the bits appended to the cache
    const float ri = wave_rinv<4>(xr, A.eps);
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = nrm(xr[k], ri, wr[k]);
    wave_rope<4>(y, rope, cs, sn);
#pragma unroll
    for (int k = 0; k < 4; ++k) sh.knb[lane + 64 * k] = f32_to_bf16(y[k]);
  }
  if (tid < QSA_D) {
    opaque(vt_raw);
    sh.vnb[tid] = f32_to_bf16(Act<T>::load(&vt_raw, 0));
  }
  __syncthreads();
  QM_PHASE(3);

  // ---- scores of keys 0..p: S^T = K Q^T with column 0 the query's hi part
  // and column 1 its lo part (the other columns zero); lane col 0 adds lane
  // col 1 (DPP row shift by 1)
  bf16x8_t qf[8];
#pragma unroll
  for (int sk = 0; sk < 8; ++sk) {
    const bf16x8_t z = {};
    qf[sk] = col < 2 ? *reinterpret_cast<const bf16x8_t*>(&sh.qb[col & 1][32 * sk + 8 * quad]) : z;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = wv + SL_WAVES * i, r16 = 16 * t;
    if (t < n_tiles) {
      if (p >= r16 && p < r16 + 16) {
        // the token's key (not yet in its page) replaces its row
        const bool krow = col == (p & 15);
#pragma unroll
        for (int sk = 0; sk < 8; ++sk) {
          const bf16x8_t kv = *reinterpret_cast<const bf16x8_t*>(&sh.knb[32 * sk + 8 * quad]);
          kf[i][sk] = krow ? kv : kf[i][sk];
        }
      }
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sk = 0; sk < 8; ++sk) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[i][sk], qf[sk], c, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float full = c[v] + row_shl<1>(c[v]);
        const int tok = r16 + 4 * quad + v;
        if (col == 0) sh.s[tok] = tok < n_tok ? full * (1.0f / 16.0f) : -INFINITY;
      }
    }
  }
  QM_PHASE(4);
  __syncthreads();
  QM_PHASE(5);

  // ---- softmax over the n_tok scores (at most one key per thread): the
  // maximum behind one barrier; each thread's weight e^(s - max) goes into its
  // wave's sum, and the PV operand forms the same weights from the scores
  const float sv = tid < n_tok ? sh.s[tid] : -INFINITY;
  float mx = wave_max(sv);
  if (lane == 0) sh.wred[wv] = mx;
  __syncthreads();
  mx = sh.wred[0];
#pragma unroll
  for (int w = 1; w < SL_WAVES; ++w) mx = fmaxf(mx, sh.wred[w]);
  const float lw = wave_sum(tid < n_tok ? __expf(sv - mx) : 0.f);
  QM_PHASE(6);

  // ---- O^T[d][0] = V^T[d][tok] P^T[tok][0] for the slice's two 16-channel
  // blocks over the wave's 32-key group; the weights as bf16 in the PV MFMA's
  // k order (e < 4: key 4 quad + e, else 16 + 4 quad + e - 4)
  f32x4_t o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  if (wv < n_grp) {
    const int r32 = 32 * wv;
    if (p >= r32 && p < r32 + 32) {
      // the token's value replaces its slot (one element of the lanes whose
      // octet holds the slot)
      const int kappa = v_slot(p - r32);
      const int dw = (kappa & 7) >> 1, sh16 = 16 * (kappa & 1);
      const bool vcol = quad == (kappa >> 3);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const unsigned val = sh.vnb[16 * (2 * cb + j) + col];
        u32x4_t u = __builtin_bit_cast(u32x4_t, vf[j]);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          if (vcol && jj == dw) u[jj] = (u[jj] & ~(0xffffu << sh16)) | (val << sh16);
        vf[j] = __builtin_bit_cast(bf16x8_t, u);
      }
    }
    float pw[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = r32 + (e < 4 ? 4 * quad + e : 16 + 4 * quad + e - 4);
      pw[e] = col == 0 && tok < n_tok ? __expf(sh.s[tok] - mx) : 0.f;
    }
    u32x4_t pu;
#pragma unroll
    for (int k = 0; k < 4; ++k) pu[k] = pack_bf16x2(pw[2 * k], pw[2 * k + 1]);
    const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, pu);
#pragma unroll
    for (int j = 0; j < 2; ++j) o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[j], pf, o[j], 0, 0, 0);
  }
  QM_PHASE(7);
  // lane (0, quad) holds channels 16 j + 4 quad + v of the slice
  if (col == 0) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) sh.red[wv][16 * j + 4 * quad + v] = o[j][v];
  }
  if (lane == 0) sh.wsum[wv] = lw;
  __syncthreads();
  if (tid < 32) {
    float num = 0.f, lsum = 0.f;
#pragma unroll
    for (int w = 0; w < SL_WAVES; ++w) {
      num += sh.red[w][tid];
      lsum += sh.wsum[w];
    }
    const float gate = Act<T>::load(&gt_raw, 0);
    Act<T>::store(out, tid, Act<T>::round(num / lsum) * Act<T>::round(sigmoid_f(gate)));
  }
  if (x == 0 && tid < QSA_D) {
    // the token's key and value into its page slot
    const int pg_cur = sh.pages[p / A.page_size], prow = p % A.page_size;
    const long cbase = pg_cur * page_stride + head_base;
    A.k_pool[cbase + k_page_index(prow, tid)] = sh.knb[tid];
    A.v_pool[cbase + v_page_index(prow, tid)] = sh.vnb[tid];
  }
  QM_PHASE(8);
  QM_PHASE_FLUSH();
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
  const long waves = (long)g->batch * seq * (g->n_heads + g->n_kv_heads + g->idx_heads);
  const long n_wg = (long)g->batch * prep_pool_per_seq(seq, g->ratio) + (waves + PREP_NT / 64 - 1) / (PREP_NT / 64);
  if (n_wg > 0x7fffffffL || waves > 0x7fffffffL) return qm_fail(QM_ERR_ARG, "qm_qsa_prep: too many rows");
  hipLaunchKernelGGL(qsa_prep_kernel<T>, dim3(static_cast<unsigned>(n_wg)), dim3(PREP_NT), 0, stream, A);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

// the several-rows block scores of batch x seq rows into scores [row][max_blocks]
int launch_score_rows(const qm_qsa_geom* g, int seq, const float* iq, const float* block_keys, const int* positions,
                      float* scores, bool fill, hipStream_t stream) {
  if ((seq + SCR_ROWS - 1) / SCR_ROWS > 65535) return qm_fail(QM_ERR_UNSUPPORTED, "qsa: more than 262140 rows");
  ScoreRowsArgs A{iq, block_keys, positions, scores, seq, g->idx_heads, g->ratio, g->max_blocks, fill ? 1 : 0};
  const dim3 grid((g->max_blocks + SCR_BLK - 1) / SCR_BLK, (seq + SCR_ROWS - 1) / SCR_ROWS, g->batch);
  hipLaunchKernelGGL(qsa_score_rows_kernel, grid, dim3(64 * SCR_ROWS), 0, stream, A);
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

QM_PHASE_ENTRY(qsa)

extern "C" int qm_v_slot(int row) { return v_slot(row); }

extern "C" int qm_qsa_page_index(int page_size, int head_dim, int* k_index, int* v_index) {
  if (page_size <= 0 || page_size % 32 || head_dim != QSA_D || !k_index || !v_index)
    return qm_fail(QM_ERR_ARG, "qm_qsa_page_index: page_size must be a multiple of 32 and head_dim 256");
  for (int r = 0; r < page_size; ++r)
    for (int d = 0; d < head_dim; ++d) {
      k_index[r * head_dim + d] = k_page_index(r, d);
      v_index[r * head_dim + d] = v_page_index(r, d);
    }
  return QM_OK;
}

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
  if (scores_out) {
    // with a score buffer the scores come from their own launch over every
    // compute unit (in the several-rows order for several rows, the one-row
    // order for one), and the selection ranks them
    if (seq > 1) {
      rc = launch_score_rows(g, seq, iq, block_keys, positions, scores_out, true, stream);
      if (rc) return rc;
    } else {
      ScoreRowArgs S{iq, block_keys, positions, scores_out, g->idx_heads, g->ratio, g->max_blocks};
      hipLaunchKernelGGL(qsa_score_row_kernel, dim3((g->max_blocks + SC1_BLK - 1) / SC1_BLK, g->batch),
                         dim3(SC1_NT), 0, stream, S);
      QM_CHECK_LAUNCH();
    }
    A.scores_in = scores_out;
    A.scores_out = nullptr;
  }
  hipLaunchKernelGGL(qsa_select_kernel, dim3(g->batch * seq), dim3(SELP_NT), 0, stream, A);
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

namespace {
struct ChunkWs {
  size_t tab, tab_bytes, o, ml, total;
};

// the slot table first: every call leaves it zero, so a workspace sized for
// a longer chunk serves a shorter one
ChunkWs chunk_ws_layout(const qm_qsa_geom* g, int seq) {
  const int nslot = g->budget / g->ratio + 1;
  const size_t rows = (size_t)g->batch * seq;
  ChunkWs w;
  w.tab = 0;
  w.tab_bytes = qm_align256((size_t)g->batch * g->max_blocks * seq * sizeof(uint16_t));
  w.o = w.tab + w.tab_bytes;
  // the partials' space first holds the rows' block scores, which the
  // selection reads before the attention writes partials over them
  const size_t o_bytes = rows * g->n_kv_heads * nslot * GQA * QSA_D * sizeof(uint16_t);
  const size_t score_bytes = rows * g->max_blocks * sizeof(float);
  w.ml = w.o + qm_align256(o_bytes > score_bytes ? o_bytes : score_bytes);
  w.total = w.ml + qm_align256(rows * g->n_kv_heads * nslot * GQA * 2 * sizeof(float));
  return w;
}

int check_chunk_geom(const qm_qsa_geom* g, const char* who) {
  int rc = check_geom(g, who);
  if (rc) return rc;
  if (g->ratio != 32 && g->ratio != 64)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_attend_chunk: indexer ratio must be 32 or 64");
  if (g->max_blocks > CA_MAX_BLOCKS || g->max_ctx > CA_MAX_BLOCKS * g->ratio)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_attend_chunk: more than 4096 blocks");
  if (g->budget / g->ratio + 1 > 511) return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_attend_chunk: top-k above 510");
  return QM_OK;
}
}  // namespace

extern "C" size_t qm_qsa_attend_chunk_workspace(const qm_qsa_geom* g, int seq) {
  if (!g || g->ratio <= 0 || g->budget < g->ratio || seq <= 0 || g->batch <= 0 || g->max_blocks <= 0) return 0;
  return chunk_ws_layout(g, seq).total;
}

namespace {
int attend_chunk(const qm_qsa_geom* g, int seq, const void* q, const void* qg, const void* k_pool, const void* v_pool,
                 const int* positions, const int* page_table, const int* ids, const int* n_sel, void* out,
                 void* workspace, size_t workspace_bytes, bool filed, hipStream_t stream) {
  int rc = check_chunk_geom(g, "qm_qsa_attend_chunk: null geometry");
  if (rc) return rc;
  if (!q || !qg || !k_pool || !v_pool || !positions || !page_table || (!filed && (!ids || !n_sel)) || !out)
    return qm_fail(QM_ERR_ARG, "qm_qsa_attend_chunk: null pointer");
  if (seq <= 0 || seq > 65535 || (long)g->batch * seq > 65535)
    return qm_fail(QM_ERR_ARG, "qm_qsa_attend_chunk: bad seq");
  const ChunkWs L = chunk_ws_layout(g, seq);
  if (!workspace || workspace_bytes < L.total)
    return qm_fail(QM_ERR_WORKSPACE, "qm_qsa_attend_chunk: workspace too small");
  char* base = static_cast<char*>(workspace);
  const int topk = g->budget / g->ratio;
  const int nslot = topk + 1;
  uint16_t* tab = reinterpret_cast<uint16_t*>(base + L.tab);
  uint16_t* part_o = reinterpret_cast<uint16_t*>(base + L.o);
  float* part_ml = reinterpret_cast<float*>(base + L.ml);

  if (!filed) {
    ChunkBucketArgs K{positions, ids, n_sel, part_ml, tab, g->batch, seq, g->n_kv_heads, g->ratio, topk, g->max_blocks};
    hipLaunchKernelGGL(qsa_chunk_bucket_kernel, dim3(g->batch * seq), dim3(64), 0, stream, K);
    QM_CHECK_LAUNCH();
  }

  ChunkAttnArgs A;
  A.q = static_cast<const uint16_t*>(q); A.k_pool = static_cast<const uint16_t*>(k_pool);
  A.v_pool = static_cast<const uint16_t*>(v_pool); A.positions = positions; A.page_table = page_table;
  A.part_o = part_o; A.part_ml = part_ml; A.tab = tab;
  A.batch = g->batch; A.seq = seq; A.hq = g->n_heads; A.hkv = g->n_kv_heads; A.page_size = g->page_size;
  A.max_pages = g->max_pages; A.ratio = g->ratio; A.topk = topk; A.max_blocks = g->max_blocks;
  A.scale = 1.0f / 16.0f;   // 1/sqrt(256), exact
  // one block per workgroup: more workgroups in flight beat blocks
  // pipelined within one (measured at 512 blocks x 2 kv heads: 31.5 us, two
  // blocks per workgroup 33.4 us, four 47.0 us)
  A.nwg_sel = g->max_blocks;
  const int n_tail = (seq + CA_TAIL_ROWS - 1) / CA_TAIL_ROWS;
  hipLaunchKernelGGL(qsa_chunk_attend_kernel, dim3(A.nwg_sel + n_tail, g->n_kv_heads, g->batch), dim3(CA_NT),
                     0, stream, A);
  QM_CHECK_LAUNCH();
  if (g->act_dtype == QM_ACT_F32) {
    CombineArgs<float, uint16_t> C{part_o, part_ml, static_cast<const float*>(qg), static_cast<float*>(out), g->n_heads,
                         g->n_kv_heads, nslot, tab, (long)(L.tab_bytes / 16)};
    hipLaunchKernelGGL((qsa_combine_kernel<float, uint16_t>), dim3(g->n_heads, g->batch * seq), dim3(QSA_D), 0, stream, C);
  } else {
    CombineArgs<bf16_t, uint16_t> C{part_o, part_ml, static_cast<const bf16_t*>(qg), static_cast<bf16_t*>(out), g->n_heads,
                          g->n_kv_heads, nslot, tab, (long)(L.tab_bytes / 16)};
    hipLaunchKernelGGL((qsa_combine_kernel<bf16_t, uint16_t>), dim3(g->n_heads, g->batch * seq), dim3(QSA_D), 0, stream, C);
  }
  QM_CHECK_LAUNCH();
  return QM_OK;
}
}  // namespace

extern "C" int qm_qsa_attend_chunk(const qm_qsa_geom* g, int seq, const void* q, const void* qg, const void* k_pool,
                                   const void* v_pool, const int* positions, const int* page_table, const int* ids,
                                   const int* n_sel, void* out, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
  return attend_chunk(g, seq, q, qg, k_pool, v_pool, positions, page_table, ids, n_sel, out, workspace,
                      workspace_bytes, false, stream);
}

extern "C" int qm_qsa_select_chunk(const qm_qsa_geom* g, int seq, const float* iq, const float* block_keys,
                                   const int* positions, int* ids, int* n_sel, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  int rc = check_chunk_geom(g, "qm_qsa_select_chunk: null geometry");
  if (rc) return rc;
  if (!iq || !block_keys || !positions || !ids || !n_sel) return qm_fail(QM_ERR_ARG, "qm_qsa_select_chunk: null pointer");
  if (seq <= 0 || seq > 65535 || (long)g->batch * seq > 65535)
    return qm_fail(QM_ERR_ARG, "qm_qsa_select_chunk: bad seq");
  if (g->max_pages > SEL_MAX_BLOCKS || g->budget / g->ratio > SEL_MAX_BLOCKS / 2)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_select_chunk: more than 4096 blocks or pages");
  const ChunkWs L = chunk_ws_layout(g, seq);
  if (!workspace || workspace_bytes < L.total)
    return qm_fail(QM_ERR_WORKSPACE, "qm_qsa_select_chunk: workspace too small");
  char* base = static_cast<char*>(workspace);
  SelArgs A = sel_args(g, seq, iq, block_keys, positions, nullptr, ids, n_sel, nullptr, nullptr);
  if (seq > 1) {
    float* scores = reinterpret_cast<float*>(base + L.o);
    rc = launch_score_rows(g, seq, iq, block_keys, positions, scores, false, stream);
    if (rc) return rc;
    A.scores_in = scores;
  }
  A.tab = reinterpret_cast<uint16_t*>(base + L.tab);
  A.part_ml = reinterpret_cast<float*>(base + L.ml);
  A.hkv = g->n_kv_heads;
  hipLaunchKernelGGL(qsa_select_kernel, dim3(g->batch * seq), dim3(SELP_NT), 0, stream, A);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

extern "C" int qm_qsa_attend_chunk_filed(const qm_qsa_geom* g, int seq, const void* q, const void* qg,
                                         const void* k_pool, const void* v_pool, const int* positions,
                                         const int* page_table, void* out, void* workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
  // the entry lists come from qm_qsa_select_chunk: no ids or counts to read
  return attend_chunk(g, seq, q, qg, k_pool, v_pool, positions, page_table, nullptr, nullptr, out, workspace,
                      workspace_bytes, true, stream);
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
  // item counts are not monotone in the position (the tail shrinks when a
  // block completes): take the largest over the last `ratio` positions, which
  // bounds every earlier one since the selected count never decreases
  int items = 1;
  for (int p = max_position - g->ratio < 0 ? 0 : max_position - g->ratio; p <= max_position; ++p) {
    const int n = items_at(g, p);
    items = n > items ? n : items;
  }
  return items < DEC_MAX_ITEMS ? items : DEC_MAX_ITEMS;
}

namespace {
// workspace of qm_qsa_decode, per (sequence, kv head) group: a generation word
// and a give-up counter (one cache line), the items' flags, their (max, sum)
// and their unnormalised outputs
size_t dec_gen_bytes(const qm_qsa_geom* g) {
  return qm_align256((size_t)g->batch * g->n_kv_heads * DEC_GEN_STRIDE * sizeof(unsigned));
}
size_t dec_flag_bytes(const qm_qsa_geom* g, int splits) {
  return qm_align256((size_t)g->batch * g->n_kv_heads * dec_flag_stride(splits) * sizeof(unsigned));
}
size_t dec_ml_bytes(const qm_qsa_geom* g, int splits) {
  return qm_align256((size_t)g->batch * g->n_kv_heads * splits * GQA * 2 * sizeof(float));
}
size_t dec_o_bytes(const qm_qsa_geom* g, int splits) {
  return qm_align256((size_t)g->batch * g->n_kv_heads * splits * GQA * QSA_D * sizeof(uint16_t));
}
}  // namespace

namespace {
const void* dec_kernel(int act_dtype, bool wide) {
  if (act_dtype == QM_ACT_F32)
    return wide ? reinterpret_cast<const void*>(&qsa_decode_kernel<float, true>)
                : reinterpret_cast<const void*>(&qsa_decode_kernel<float, false>);
  return wide ? reinterpret_cast<const void*>(&qsa_decode_kernel<bf16_t, true>)
              : reinterpret_cast<const void*>(&qsa_decode_kernel<bf16_t, false>);
}
}  // namespace

extern "C" int qm_qsa_decode_group(int splits) { return splits < DEC_SLICES ? DEC_SLICES : splits; }

extern "C" int qm_qsa_decode_fits(int splits, int resident) {
  if (splits <= 0 || splits > DEC_MAX_ITEMS)
    return qm_fail(QM_ERR_ARG, "qm_qsa_decode: splits must be 1..1024 (qm_qsa_decode_splits)");
  if (qm_qsa_decode_group(splits) > resident)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_decode: a (sequence, kv head) group of this many workgroups cannot "
                                       "be resident on the device at once (use qm_qsa_decode_front + "
                                       "qm_qsa_attend)");
  return QM_OK;
}

extern "C" int qm_qsa_decode_resident(int act_dtype, int splits) {
  if (act_dtype != QM_ACT_F32 && act_dtype != QM_ACT_BF16)
    return qm_fail(QM_ERR_DTYPE, "qm_qsa_decode_resident: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
  int v = 0;
  const int rc = qm_resident_workgroups(dec_kernel(act_dtype, splits < DEC_SLICES), DEC_NT, 0, &v);
  return rc ? rc : v;
}

extern "C" int qm_qsa_decode_check(const qm_qsa_geom* g, int splits, void* workspace, size_t workspace_bytes,
                                   int reset, unsigned* counts, hipStream_t stream) {
  int rc = check_geom(g, "qm_qsa_decode_check: null geometry");
  if (rc) return rc;
  if (!workspace || !counts) return qm_fail(QM_ERR_ARG, "qm_qsa_decode_check: null pointer");
  if (splits <= 0 || workspace_bytes < qm_qsa_decode_workspace(g, splits))
    return qm_fail(QM_ERR_WORKSPACE, "qm_qsa_decode_check: workspace too small for these splits");
  const long n_groups = (long)g->batch * g->n_kv_heads;
  unsigned* lines = static_cast<unsigned*>(workspace);
  unsigned* host = new unsigned[n_groups * DEC_GEN_STRIDE];
  hipError_t e = hipMemcpyAsync(host, lines, n_groups * DEC_GEN_STRIDE * sizeof(unsigned), hipMemcpyDeviceToHost,
                                stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    delete[] host;
    return qm_fail(QM_ERR_LAUNCH, hipGetErrorString(e));
  }
  counts[0] = counts[1] = 0;
  for (long i = 0; i < n_groups; ++i) {
    counts[0] += host[i * DEC_GEN_STRIDE + 1];
    counts[1] += host[i * DEC_GEN_STRIDE + 2];
  }
  delete[] host;
  if (!reset) return QM_OK;
  // generation words, counters and flags back to zero: the state of a fresh workspace
  const size_t words = (dec_gen_bytes(g) + dec_flag_bytes(g, splits)) / sizeof(unsigned);
  return qm_zero_words(workspace, (long)words, stream);
}

extern "C" size_t qm_qsa_decode_workspace(const qm_qsa_geom* g, int splits) {
  if (!g || splits <= 0) return 0;
  return dec_gen_bytes(g) + dec_flag_bytes(g, splits) + dec_ml_bytes(g, splits) + dec_o_bytes(g, splits);
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
  if (g->max_blocks > DEC_MAX_BLOCKS || g->max_pages > DEC_MAX_PAGES || g->budget / g->ratio > DEC_MAX_TOPK ||
      g->ratio > DEC_MAX_RATIO)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_qsa_decode: more than 2048 blocks or pages, top-k above 256 or ratio "
                                       "above 64 (use qm_qsa_prep + qm_qsa_select + qm_qsa_attend)");
  if (splits <= 0 || splits > DEC_MAX_ITEMS)
    return qm_fail(QM_ERR_ARG, "qm_qsa_decode: splits must be 1..1024 (qm_qsa_decode_splits)");
  if (g->batch > 65535) return qm_fail(QM_ERR_ARG, "qm_qsa_decode: batch above 65535");
  if (!workspace || workspace_bytes < qm_qsa_decode_workspace(g, splits))
    return qm_fail(QM_ERR_WORKSPACE, "qm_qsa_decode: workspace too small");
  char* ws = static_cast<char*>(workspace);
  unsigned* gen = reinterpret_cast<unsigned*>(ws);
  // Short contexts (a plan of at most SL_FAST_ITEMS attention items, so at most
  // 32 SL_FAST_ITEMS keys, with a budget that keeps the selection off for all
  // of them) take the slice kernel: no workgroup waits for another.
  if (splits <= SL_FAST_ITEMS && g->budget >= SL_MAX_TOK) {
    const dim3 grid(DEC_SLICES + 1, g->n_kv_heads, g->batch);
    auto run_slices = [&](auto* tag) -> int {
      using T = std::remove_pointer_t<decltype(tag)>;
      DecArgs<T> D{};
      D.P = prep_args<T>(g, 1, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos, sin, positions,
                         page_table, k_pool, v_pool, raw_keys, block_keys, nullptr, nullptr);
      D.gen = gen; D.out = static_cast<T*>(out);
      D.ids = ids; D.n_sel = n_sel; D.items = static_cast<int2*>(items); D.iq_out = iq_out;
      D.splits = splits; D.topk = g->budget / g->ratio; D.max_items = item_stride(g);
      hipLaunchKernelGGL(qsa_decode_slices_kernel<T>, grid, dim3(SL_NT), 0, stream, D);
      QM_CHECK_LAUNCH();
      return QM_OK;
    };
    if (g->act_dtype == QM_ACT_F32) return run_slices(static_cast<float*>(nullptr));
    return run_slices(static_cast<bf16_t*>(nullptr));
  }
  // every workgroup of a (sequence, kv head) group waits for the others: the
  // group must fit on the device at once (groups are dispatched in order, so
  // one group at a time is enough)
  const int resident = qm_qsa_decode_resident(g->act_dtype, splits);
  if (resident < 0) return resident;
  rc = qm_qsa_decode_fits(splits, resident);
  if (rc) return rc;
  unsigned* flags = reinterpret_cast<unsigned*>(ws + dec_gen_bytes(g));
  float* part_ml = reinterpret_cast<float*>(ws + dec_gen_bytes(g) + dec_flag_bytes(g, splits));
  uint16_t* part_o = reinterpret_cast<uint16_t*>(ws + dec_gen_bytes(g) + dec_flag_bytes(g, splits) + dec_ml_bytes(g, splits));
  const bool wide = splits < DEC_SLICES;
  const dim3 grid(wide ? DEC_SLICES : splits, g->n_kv_heads, g->batch);
  auto run = [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    DecArgs<T> D;
    D.P = prep_args<T>(g, 1, qg, k_new, v_new, iq, ik, q_norm, k_norm, iq_norm, ik_norm, cos, sin, positions,
                       page_table, k_pool, v_pool, raw_keys, block_keys, nullptr, nullptr);
    D.part_o = part_o; D.part_ml = part_ml; D.gen = gen; D.flags = flags; D.out = static_cast<T*>(out);
    D.ids = ids; D.n_sel = n_sel; D.items = static_cast<int2*>(items); D.iq_out = iq_out;
    D.splits = splits; D.topk = g->budget / g->ratio; D.max_items = item_stride(g);
    const int gpb = g->ratio >= 32 ? g->ratio / 32 : 1;
    const unsigned may_score = splits > D.topk * gpb ? 1u : 0u;
    const unsigned dims0 = (unsigned)g->max_blocks | ((unsigned)g->rope_dim << 16) |
                           ((unsigned)g->idx_heads << 24) | (may_score << 28);
    const unsigned dims1 = (unsigned)__builtin_ctz((unsigned)g->ratio) | ((unsigned)D.topk << 8);
    const T* iq_t = static_cast<const T*>(iq);
    if (wide)
      hipLaunchKernelGGL((qsa_decode_kernel<T, true>), grid, dim3(DEC_NT), 0, stream, positions, iq_t, iq_norm,
                         static_cast<const float*>(block_keys), cos, sin, dims0, dims1, D);
    else
      hipLaunchKernelGGL((qsa_decode_kernel<T, false>), grid, dim3(DEC_NT), 0, stream, positions, iq_t, iq_norm,
                         static_cast<const float*>(block_keys), cos, sin, dims0, dims1, D);
    QM_CHECK_LAUNCH();
    return QM_OK;
  };
  if (g->act_dtype == QM_ACT_F32) return run(static_cast<float*>(nullptr));
  return run(static_cast<bf16_t*>(nullptr));
}
