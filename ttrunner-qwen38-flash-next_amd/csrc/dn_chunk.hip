// Gated delta rule over 64-token chunks in the WY/UT form, gfx950.
//
// chunk_gated_delta_rule (reference/layers.py:195-275). The chunk-local algebra
// is independent across chunks and the state recurrence is not, so the rule
// runs as two launches:
//   dn_chunk_prep   one or four workgroups per (sequence, head, chunk): l2-normalises q
//                   and k, takes the cumulative log-decay (in double, as torch's
//                   CPU cumsum accumulates), forms L = (k beta k^T) * decay
//                   below the diagonal and (q k^T) * decay on and below it,
//                   inverts I + L (16x16 diagonal blocks by substitution, the
//                   blocks below by MFMA, one sub-diagonal at a time) and writes
//                   w = T (k beta e^cum), u = T (v beta), q e^cum and
//                   (k e^(cum_last - cum))^T to the workspace
//   dn_chunk_scan   one workgroup per (sequence, head, 16 columns of d_v): the
//                   state slice [128 x 16] stays on chip while the chunks pass:
//                   v_new = u - w S, out = q_dec S + qk v_new,
//                   S = S e^cum_last + k_dec^T v_new
// Every product is a v_mfma_f32_16x16x4_f32 (fp32 in, fp32 accumulate); its
// operand lanes are A[row l%16][k l/16], B[k l/16][col l%16] and the result
// rows 4(l/16)+i, col l%16. K runs in the order 16j + 4(l/16) + e over float4
// operand loads, the same for both operands, so an accumulator's four rows
// feed the next product's B operand without a trip through LDS.
#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int CK_C = 64;          // tokens per chunk
constexpr int CK_D = 128;         // d_k = d_v
constexpr int CK_NT = 256;        // four waves
constexpr int CK_LD = CK_D + 4;   // LDS row stride of [token][dim] tiles, floats
constexpr int CK_LT = CK_C + 4;   // LDS row stride of [.][token] tiles, floats
constexpr int CK_COLS = 16;       // d_v columns per scan workgroup
constexpr int CK_MIN_SEQ = 16;    // shorter prefill chunks take the token loop
constexpr int CK_PARTS = 4;       // prep workgroups per chunk when chunks are few

// One fp32 record per (sequence, head, chunk):
//   w   [64][128]   T (k beta e^cum)                               fragment order
//   u   [64][128]   T (v beta)                                     row-major
//   qd  [64][128]   q e^cum (q l2-normalised and scaled by d^-1/2) fragment order
//   kdT [128][64]   (k e^(cum_last - cum))^T                       fragment order
//   qk  [64][64]    (q k^T) * decay on and below the diagonal      fragment order
//   ecl [64]        e^cum_last in element 0
// Fragment order (frag_index) stores each 16x16 block as the A operands of its
// four 16x16x4 MFMA steps in lane order: every wave-wide float4 load of the
// scan reads 1 KB of contiguous memory.
constexpr long CK_W = 0;
constexpr long CK_U = CK_W + CK_C * CK_D;
constexpr long CK_QD = CK_U + CK_C * CK_D;
constexpr long CK_KDT = CK_QD + CK_C * CK_D;
constexpr long CK_QK = CK_KDT + CK_C * CK_D;
constexpr long CK_ECL = CK_QK + CK_C * CK_C;
constexpr long CK_REC = CK_ECL + 64;
static_assert((CK_REC * 4) % 256 == 0, "records stay 256-byte aligned");

// offset of element (row, col) of a [rows][ncol] matrix in fragment order:
// 16x16 block, then lane 16 * ((col % 16) / 4) + row % 16, then col % 4
__device__ __forceinline__ int frag_index(int row, int col, int ncol) {
  return ((((row >> 4) * (ncol >> 4) + (col >> 4)) * 64 + ((col & 15) >> 2) * 16 + (row & 15)) << 2) + (col & 3);
}

__device__ __forceinline__ f32x4_t mfma4(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t mfma4x4(float4 a, float4 b, f32x4_t c) {
  c = mfma4(a.x, b.x, c);
  c = mfma4(a.y, b.y, c);
  c = mfma4(a.z, b.z, c);
  return mfma4(a.w, b.w, c);
}

__device__ __forceinline__ float4 lds4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// eight consecutive activations as float
__device__ __forceinline__ void load8(const float* p, float* o) {
  const float4 a = ld4(p), b = ld4(p + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
__device__ __forceinline__ void load8(const bf16_t* p, float* o) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = bf16_to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
    o[2 * i + 1] = bf16_to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}

// lower 16x16 tiles (I, J), J <= I, numbered (0,0) (1,0) (1,1) (2,0) ... (3,3)
__device__ __forceinline__ void tile_ij(int t, int& I, int& J) {
  I = t < 1 ? 0 : t < 3 ? 1 : t < 6 ? 2 : 3;
  J = t - I * (I + 1) / 2;
}

// 16x16 tile of X Y^T over 128 dims: a = &X[row0 + l%16][4(l/16)], b likewise
__device__ __forceinline__ f32x4_t gram_tile(const float* a, const float* b) {
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 8; ++j) acc = mfma4x4(lds4(a + 16 * j), lds4(b + 16 * j), acc);
  return acc;
}

template <typename T>
struct ChunkPrepArgs {
  const T* q; const T* k; const T* v;   // token rows of q_stride / v_stride elements
  const float* g; const float* beta;    // [B, S, H]
  float* ws;                            // [B, H, n_chunks] records
  int batch, seq, heads, hk, n_chunks;  // head h reads q/k head h % hk
  int parts;                            // workgroups per chunk: 1 or CK_PARTS
  long q_stride, v_stride;
};

struct PrepShared {
  float q[CK_C][CK_LD];    // normalised q * d^-1/2
  float k[CK_C][CK_LD];    // normalised k
  float v[CK_C][CK_LD];    // v * beta
  float L[CK_C][CK_LT];    // (k beta k^T) * decay, strictly lower
  float Tm[CK_C][CK_LT];   // (I + L)^-1, lower
  float cum[CK_C], beta[CK_C], ecum[CK_C], bec[CK_C], kds[CK_C];
};

template <typename T>
__global__ __launch_bounds__(CK_NT) void dn_chunk_prep_kernel(ChunkPrepArgs<T> A) {
  __shared__ PrepShared sh;
  QM_PHASE_DECL
  QM_PHASE(0);
  // A.parts workgroups per chunk: each forms L and T, then writes its share
  // (all of it, or a quarter) of qk, q_dec, k_dec^T and of the w / u columns
  const int part = blockIdx.x % A.parts;
  const int c = (blockIdx.x / A.parts) % A.n_chunks;
  const int bh = blockIdx.x / A.parts / A.n_chunks;
  const int span = CK_PARTS / A.parts;       // quarters this workgroup writes
  const int h = bh % A.heads, b = bh / A.heads;
  const int t0 = c * CK_C;
  const int n_valid = min(CK_C, A.seq - t0);
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int g4 = lane >> 4, r16 = lane & 15;
  float* rec = A.ws + ((long)bh * A.n_chunks + c) * CK_REC;

  // gates; padding tokens carry g = 0 and beta = 0
  if (wid == 0) {
    const bool ok = lane < n_valid;
    const long gi = ((long)b * A.seq + t0 + (ok ? lane : 0)) * A.heads + h;
    const float gv = ok ? A.g[gi] : 0.f;
    const float bv = ok ? A.beta[gi] : 0.f;
    double s = gv;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double o = __shfl_up(s, off, 64);
      if (lane >= off) s += o;
    }
    const float cum = static_cast<float>(s);
    const float last = __shfl(cum, 63, 64);
    const float ec = expf(cum);
    sh.cum[lane] = cum;
    sh.beta[lane] = bv;
    sh.ecum[lane] = ec;
    sh.bec[lane] = bv * ec;
    sh.kds[lane] = expf(last - cum);
    if (lane == 0 && part == 0) rec[CK_ECL] = expf(last);
  }

  // q, k, v rows: four threads per token, 32 dims each as four runs of 8
  {
    const int t = tid >> 2, p = tid & 3;
    const bool ok = t < n_valid;
    const long tok = (long)b * A.seq + t0 + (ok ? t : 0);
    const long qo = tok * A.q_stride + (long)(h % A.hk) * CK_D;
    const long vo = tok * A.v_stride + (long)h * CK_D;
    const float bv = ok ? A.beta[tok * A.heads + h] : 0.f;
    float qv[32], kv[32], vv[32];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 8 * (p + 4 * j);
      load8(A.q + qo + d, qv + 8 * j);
      load8(A.k + qo + d, kv + 8 * j);
      load8(A.v + vo + d, vv + 8 * j);
    }
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      sq = fmaf(qv[i], qv[i], sq);
      sk = fmaf(kv[i], kv[i], sk);
    }
    sq += __shfl_xor(sq, 1, 64);
    sk += __shfl_xor(sk, 1, 64);
    sq += __shfl_xor(sq, 2, 64);
    sk += __shfl_xor(sk, 2, 64);
    const float rq = ok ? rsqrt_rn(sq + 1e-6f) : 0.f;
    const float rk = ok ? rsqrt_rn(sk + 1e-6f) : 0.f;
    const float qscale = 0.08838834764831845f;  // 128^-1/2
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 8; e += 4) {
        const int d = 8 * (p + 4 * j) + e;
        const float* x = qv + 8 * j + e;
        const float* y = kv + 8 * j + e;
        const float* z = vv + 8 * j + e;
        *reinterpret_cast<float4*>(&sh.q[t][d]) =
            make_float4(mul_rn(mul_rn(x[0], rq), qscale), mul_rn(mul_rn(x[1], rq), qscale),
                        mul_rn(mul_rn(x[2], rq), qscale), mul_rn(mul_rn(x[3], rq), qscale));
        *reinterpret_cast<float4*>(&sh.k[t][d]) =
            make_float4(mul_rn(y[0], rk), mul_rn(y[1], rk), mul_rn(y[2], rk), mul_rn(y[3], rk));
        *reinterpret_cast<float4*>(&sh.v[t][d]) = make_float4(z[0] * bv, z[1] * bv, z[2] * bv, z[3] * bv);
      }
    }
  }
  QM_PHASE(1);
  __syncthreads();
  QM_PHASE(2);

  // L = (k k^T) * beta_i * exp(cum_i - cum_j) for j < i
  for (int ti = wid; ti < 10; ti += 4) {
    int I, J;
    tile_ij(ti, I, J);
    const f32x4_t acc = gram_tile(&sh.k[16 * I + r16][4 * g4], &sh.k[16 * J + r16][4 * g4]);
    const int j = 16 * J + r16;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 16 * I + 4 * g4 + v;
      sh.L[i][j] = i > j ? (acc[v] * sh.beta[i]) * expf(sh.cum[i] - sh.cum[j]) : 0.f;
    }
  }
  QM_PHASE(3);
  __syncthreads();
  QM_PHASE(4);

  if (wid == 0) {
    // (I + L_II)^-1 for the four diagonal blocks; lane = (block, column):
    // x_i = [i == col] - sum_{k<i} L_ik x_k
    const int I = g4, col = r16;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float* Lr = &sh.L[16 * I + i][16 * I];
      float acc = i == col ? 1.f : 0.f;
#pragma unroll
      for (int kk = 0; kk < i; ++kk) acc = fmaf(-Lr[kk], x[kk], acc);
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sh.Tm[16 * I + i][16 * I + col] = x[i];
  } else {
    // qk = (q k^T) * exp(cum_i - cum_j) for j <= i: tile ti belongs to quarter
    // ti % 4; this workgroup's tiles go round-robin to waves 1-3
    int k = 0;
    for (int ti = 0; ti < 10; ++ti) {
      if ((ti & 3) / span != part) continue;
      if (k++ % 3 != wid - 1) continue;
      int I, J;
      tile_ij(ti, I, J);
      const f32x4_t acc = gram_tile(&sh.q[16 * I + r16][4 * g4], &sh.k[16 * J + r16][4 * g4]);
      const int j = 16 * J + r16;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * I + 4 * g4 + v;
        rec[CK_QK + frag_index(i, j, CK_C)] = i >= j ? acc[v] * expf(sh.cum[i] - sh.cum[j]) : 0.f;
      }
    }
  }

  QM_PHASE(5);
  // q e^cum as [token][dim] and (k e^(cum_last - cum))^T as [dim][token]
  for (int it = 2 * span * part; it < 2 * span * (part + 1); ++it) {
    const int idx = tid + CK_NT * it;
    const int t = idx >> 5, d = 4 * (idx & 31);
    const float4 x = lds4(&sh.q[t][d]);
    const float e = sh.ecum[t];
    *reinterpret_cast<float4*>(rec + CK_QD + frag_index(t, d, CK_D)) = make_float4(x.x * e, x.y * e, x.z * e, x.w * e);
  }
  for (int it = 2 * span * part; it < 2 * span * (part + 1); ++it) {
    const int idx = tid + CK_NT * it;
    const int t = 4 * (idx & 15), d = idx >> 4;
    *reinterpret_cast<float4*>(rec + CK_KDT + frag_index(d, t, CK_C)) =
        make_float4(sh.k[t][d] * sh.kds[t], sh.k[t + 1][d] * sh.kds[t + 1], sh.k[t + 2][d] * sh.kds[t + 2],
                    sh.k[t + 3][d] * sh.kds[t + 3]);
  }
  __syncthreads();

  QM_PHASE(6);
  // blocks of T below the diagonal, one sub-diagonal at a time:
  // T_IJ = -T_II sum_{K=J}^{I-1} L_IK T_KJ
  for (int dist = 1; dist < 4; ++dist) {
    if (wid < 4 - dist) {
      const int J = wid, I = wid + dist;
      f32x4_t p = {0.f, 0.f, 0.f, 0.f};
      for (int K = J; K < I; ++K) {
        const float4 a = lds4(&sh.L[16 * I + r16][16 * K + 4 * g4]);
        const float* tb = &sh.Tm[16 * K + 4 * g4][16 * J + r16];
        p = mfma4x4(a, make_float4(tb[0], tb[CK_LT], tb[2 * CK_LT], tb[3 * CK_LT]), p);
      }
      const float4 xa = lds4(&sh.Tm[16 * I + r16][16 * I + 4 * g4]);
      f32x4_t x = {0.f, 0.f, 0.f, 0.f};
      x = mfma4x4(xa, make_float4(p[0], p[1], p[2], p[3]), x);
#pragma unroll
      for (int v = 0; v < 4; ++v) sh.Tm[16 * I + 4 * g4 + v][16 * J + r16] = -x[v];
    }
    __syncthreads();
  }

  QM_PHASE(7);
  // w = T (k beta e^cum) and u = T (v beta): quarter r holds column tiles 2r
  // and 2r + 1 of each, one (matrix, tile) per wave
  for (int kq = 0; kq < span; ++kq) {
    const bool is_u = wid >= 2;
    const int col = 16 * (2 * (span * part + kq) + (wid & 1)) + r16;
    float bo[4][4];
#pragma unroll
    for (int K = 0; K < 4; ++K) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * K + 4 * g4 + e;
        bo[K][e] = is_u ? sh.v[t][col] : sh.k[t][col] * sh.bec[t];
      }
    }
    float* dst = rec + (is_u ? CK_U : CK_W);
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int K = 0; K <= I; ++K)
        acc = mfma4x4(lds4(&sh.Tm[16 * I + r16][16 * K + 4 * g4]), make_float4(bo[K][0], bo[K][1], bo[K][2], bo[K][3]),
                      acc);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * I + 4 * g4 + v;
        dst[is_u ? row * CK_D + col : frag_index(row, col, CK_D)] = acc[v];
      }
    }
  }
  QM_PHASE(8);
  QM_PHASE_FLUSH();
}

template <typename T>
struct ChunkScanArgs {
  const float* ws;   // [B, H, n_chunks] records
  float* state;      // [B, H, 128, 128]
  T* out;            // [B, S, H, 128]
  int batch, seq, heads, n_chunks;
};

// A wave's operands of one chunk, none of which depends on the state: its 16
// rows of w and q_dec, its row block of qk (blocks j <= wave used), its two
// 16-row blocks of k_dec^T, its 4 values of u, and e^cum_last.
struct ScanOps {
  float4 w[8], qd[8], qk[4], kd[2][4];
  float u[4], ecl;
};

__device__ __forceinline__ void load_scan_ops(const float* rec, int wid, int g4, int r16, int col0, ScanOps& o) {
  const int lane4 = (16 * g4 + r16) * 4;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    o.w[j] = ld4(rec + CK_W + (wid * 8 + j) * 256 + lane4);
    o.qd[j] = ld4(rec + CK_QD + (wid * 8 + j) * 256 + lane4);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) o.qk[j] = ld4(rec + CK_QK + (wid * 4 + j) * 256 + lane4);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) o.kd[t][j] = ld4(rec + CK_KDT + ((2 * wid + t) * 4 + j) * 256 + lane4);
  const float* ur = rec + CK_U + (16 * wid + 4 * g4) * CK_D + col0 + r16;
#pragma unroll
  for (int v = 0; v < 4; ++v) o.u[v] = ur[v * CK_D];
  o.ecl = rec[CK_ECL];
}

template <typename T>
__global__ __launch_bounds__(CK_NT) void dn_chunk_scan_kernel(ChunkScanArgs<T> A) {
  __shared__ float sST[CK_COLS][CK_LD];  // the state slice, transposed: [column][d_k]
  __shared__ float sVT[CK_COLS][CK_LT];  // v_new of the chunk, transposed: [column][token]
  QM_PHASE_DECL
  QM_PHASE(0);
  constexpr int NSL = CK_D / CK_COLS;
  const int nwg = A.batch * A.heads * NSL;
  const int wg = xcd_remap(blockIdx.x, nwg);
  const int sl = wg % NSL, bh = wg / NSL;
  const int h = bh % A.heads, b = bh / A.heads;
  const int col0 = sl * CK_COLS;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int g4 = lane >> 4, r16 = lane & 15;
  const float* recs = A.ws + (long)bh * A.n_chunks * CK_REC;

  // operands two chunks ahead: three register sets, the loop unrolled by
  // three so that no set is copied while its loads are in flight
  ScanOps o0, o1, o2;
  load_scan_ops(recs, wid, g4, r16, col0, o0);
  load_scan_ops(recs + (long)min(1, A.n_chunks - 1) * CK_REC, wid, g4, r16, col0, o1);
  // wave wid keeps d_k rows 32wid .. 32wid+31 of the slice as two result tiles
  float* S = A.state + (long)bh * CK_D * CK_D + col0 + r16;
  f32x4_t st[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int row = 32 * wid + 16 * t + 4 * g4;
#pragma unroll
    for (int v = 0; v < 4; ++v) st[t][v] = S[(long)(row + v) * CK_D];
    *reinterpret_cast<float4*>(&sST[r16][row]) = make_float4(st[t][0], st[t][1], st[t][2], st[t][3]);
  }

  QM_PHASE(1);
  auto chunk = [&](int ci, const ScanOps& cur, ScanOps& ahead) {
    // chunk ci + 2's operands fly during this one (clamped at the last chunk)
    load_scan_ops(recs + (long)min(ci + 2, A.n_chunks - 1) * CK_REC, wid, g4, r16, col0, ahead);
    __syncthreads();
    // rows 16wid.. of w S and q_dec S
    f32x4_t aw = {0.f, 0.f, 0.f, 0.f}, ao = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 sb = lds4(&sST[r16][16 * j + 4 * g4]);
      aw = mfma4x4(cur.w[j], sb, aw);
      ao = mfma4x4(cur.qd[j], sb, ao);
    }
    *reinterpret_cast<float4*>(&sVT[r16][16 * wid + 4 * g4]) =
        make_float4(cur.u[0] - aw[0], cur.u[1] - aw[1], cur.u[2] - aw[2], cur.u[3] - aw[3]);
    __syncthreads();

    // out rows 16wid..: q_dec S + qk v_new over the causal blocks j <= wid
    float4 vb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) vb[j] = lds4(&sVT[r16][16 * j + 4 * g4]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j <= wid) ao = mfma4x4(cur.qk[j], vb[j], ao);
    const int tok0 = ci * CK_C + 16 * wid + 4 * g4;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (tok0 + v < A.seq)
        Act<T>::store(A.out, (((long)b * A.seq + tok0 + v) * A.heads + h) * CK_D + col0 + r16, ao[v]);

    // S = S e^cum_last + k_dec^T v_new on this wave's rows
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = 32 * wid + 16 * t;
      f32x4_t acc = {st[t][0] * cur.ecl, st[t][1] * cur.ecl, st[t][2] * cur.ecl, st[t][3] * cur.ecl};
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = mfma4x4(cur.kd[t][j], vb[j], acc);
      st[t] = acc;
      *reinterpret_cast<float4*>(&sST[r16][row + 4 * g4]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
    if (ci < 12) QM_PHASE(2 + ci);
  };

  for (int ci = 0; ci < A.n_chunks; ci += 3) {
    chunk(ci, o0, o2);
    if (ci + 1 < A.n_chunks) chunk(ci + 1, o1, o0);
    if (ci + 2 < A.n_chunks) chunk(ci + 2, o2, o1);
  }

#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int row = 32 * wid + 16 * t + 4 * g4;
#pragma unroll
    for (int v = 0; v < 4; ++v) S[(long)(row + v) * CK_D] = st[t][v];
  }
  QM_PHASE(14);
  QM_PHASE_FLUSH_AT(4096u);
}

template <typename T>
int launch_chunked(int batch, int seq, int heads, int hk, long q_stride, long v_stride, const void* q, const void* k,
                   const void* v, const float* g, const float* beta, float* state, void* out, float* ws,
                   hipStream_t stream) {
  const int n_chunks = (seq + CK_C - 1) / CK_C;
  ChunkPrepArgs<T> P;
  P.q = static_cast<const T*>(q); P.k = static_cast<const T*>(k); P.v = static_cast<const T*>(v);
  P.g = g; P.beta = beta; P.ws = ws;
  P.batch = batch; P.seq = seq; P.heads = heads; P.hk = hk; P.n_chunks = n_chunks;
  P.q_stride = q_stride; P.v_stride = v_stride;
  // few chunks: four workgroups per chunk so that the launch fills the chip;
  // many: one each, since every workgroup repeats the L and T work
  P.parts = (long)batch * heads * n_chunks < 256 ? CK_PARTS : 1;
  hipLaunchKernelGGL(dn_chunk_prep_kernel<T>, dim3(batch * heads * n_chunks * P.parts), dim3(CK_NT), 0, stream, P);
  QM_CHECK_LAUNCH();
  ChunkScanArgs<T> S;
  S.ws = ws; S.state = state; S.out = static_cast<T*>(out);
  S.batch = batch; S.seq = seq; S.heads = heads; S.n_chunks = n_chunks;
  hipLaunchKernelGGL(dn_chunk_scan_kernel<T>, dim3(batch * heads * (CK_D / CK_COLS)), dim3(CK_NT), 0, stream, S);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

int run_chunked(int act_dtype, int batch, int seq, int heads, int hk, long q_stride, long v_stride, const void* q,
                const void* k, const void* v, const float* g, const float* beta, float* state, void* out, void* ws,
                hipStream_t stream) {
  float* w = static_cast<float*>(ws);
  if (act_dtype == QM_ACT_F32)
    return launch_chunked<float>(batch, seq, heads, hk, q_stride, v_stride, q, k, v, g, beta, state, out, w, stream);
  if (act_dtype == QM_ACT_BF16)
    return launch_chunked<bf16_t>(batch, seq, heads, hk, q_stride, v_stride, q, k, v, g, beta, state, out, w,
                                  stream);
  return qm_fail(QM_ERR_DTYPE, "delta rule: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
}

}  // namespace

QM_PHASE_ENTRY(dnc)

namespace {
size_t chunk_records_bytes(int batch, int seq, int heads) {
  if (batch <= 0 || seq <= 0 || heads <= 0) return 0;
  const size_t n_chunks = (size_t)(seq + CK_C - 1) / CK_C;
  return (size_t)batch * heads * n_chunks * CK_REC * sizeof(float);
}
}  // namespace

size_t qm_dn_rule_chunk_workspace(int batch, int seq, int heads) {
  return seq < CK_MIN_SEQ ? 0 : chunk_records_bytes(batch, seq, heads);
}

int qm_dn_rule_chunk(int act_dtype, int batch, int seq, int heads, int hk, long q_stride, long v_stride,
                     const void* q, const void* k, const void* v, const float* g, const float* beta, float* state,
                     void* out, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (seq < CK_MIN_SEQ)
    return qm_dn_recurrent_strided(act_dtype, batch, seq, heads, hk, q_stride, v_stride, q, k, v, g, beta, state, out,
                                   stream);
  if (!ws || ws_bytes < chunk_records_bytes(batch, seq, heads))
    return qm_fail(QM_ERR_WORKSPACE, "delta rule: workspace too small for the chunked form");
  return run_chunked(act_dtype, batch, seq, heads, hk, q_stride, v_stride, q, k, v, g, beta, state, out, ws, stream);
}

extern "C" size_t qm_dn_chunked_workspace(int batch, int seq, int heads, int head_dim) {
  if (head_dim != CK_D) return 0;
  return chunk_records_bytes(batch, seq, heads);
}

extern "C" int qm_dn_chunked(int act_dtype, int batch, int seq, int heads, int head_dim, const void* q, const void* k,
                             const void* v, const float* g, const float* beta, float* state, void* out,
                             void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (head_dim != CK_D) return qm_fail(QM_ERR_UNSUPPORTED, "qm_dn_chunked: head_dim must be 128");
  if (batch <= 0 || seq < 0 || heads <= 0) return qm_fail(QM_ERR_ARG, "qm_dn_chunked: bad sizes");
  if (!q || !k || !v || !g || !beta || !state || !out) return qm_fail(QM_ERR_ARG, "qm_dn_chunked: null pointer");
  if (act_dtype != QM_ACT_F32 && act_dtype != QM_ACT_BF16)
    return qm_fail(QM_ERR_DTYPE, "qm_dn_chunked: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
  if (seq == 0) return QM_OK;
  if (!workspace || workspace_bytes < chunk_records_bytes(batch, seq, heads))
    return qm_fail(QM_ERR_WORKSPACE, "qm_dn_chunked: workspace too small");
  return run_chunked(act_dtype, batch, seq, heads, heads, (long)heads * CK_D, (long)heads * CK_D, q, k, v, g, beta,
                     state, out, workspace, stream);
}
