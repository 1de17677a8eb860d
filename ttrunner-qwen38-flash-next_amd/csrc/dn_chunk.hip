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
//                   blocks below by fp32 MFMA, one sub-diagonal at a time) and
//                   writes w = T (k beta e^cum), u = T (v beta), q e^cum and
//                   k e^(cum_last - cum) to the workspace
//   dn_chunk_scan   one workgroup per (sequence, head, 16 columns of d_v): the
//                   state slice stays on chip while the chunks pass:
//                   v_new = u - w S, out = q_dec S + qk v_new,
//                   S = S e^cum_last + k_dec^T v_new
// The products over d_k and over tokens run on v_mfma_f32_16x16x32_bf16 with
// each fp32 operand split into bf16 high and low parts, x = hi + lo to 16
// significant bits: a b = hi hi + hi lo + lo hi, the lo lo term (2^-18 of the
// product) dropped, every sum accumulated in fp32. One such product costs
// three bf16 MFMAs where the same 16x16x32 product takes eight fp32
// 16x16x4 MFMAs of twice the cycles each. Operand lanes: A[row l%16][k 8(l/16)
// + e], B[k 8(l/16) + e][col l%16], e < 8; result rows 4(l/16)+i, col l%16.
// The scan works on transposed products (S^T w^T, S^T q_dec^T, v_new^T qk^T,
// v_new^T k_dec), so that the state's A operand and every record operand are
// runs of 8 consecutive elements in memory.
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

// One record per (sequence, head, chunk), in floats. A fragment pair is the
// bf16 high parts of one 16x32 MFMA operand (64 lanes x 8, 1 KB) followed by
// its low parts: FRAG2 floats. Fragment (b, s) of a matrix holds rows 16 b ..
// 16 b + 15 and k-step s (k = 32 s .. 32 s + 31) in operand lane order, so a
// wave's operand load reads 1 KB of contiguous memory.
//   W    w[tok][dk] = T (k beta e^cum)          (token block, dk step)  4 x 4
//   QD   q e^cum [tok][dk] (q l2-normalised, scaled by d^-1/2)          4 x 4
//   QK   (q k^T)[i][j] * decay, j <= i          (i block, j step)       4 x 2
//   KD   k e^(cum_last - cum), as [dk][tok]     (dk block, token step)  8 x 2
//   U    u = T (v beta) [tok][dv], fp32 row-major
//   ECL  e^cum_last in element 0
constexpr long FRAG2 = 512;
constexpr long CK_W = 0;
constexpr long CK_QD = CK_W + 16 * FRAG2;
constexpr long CK_QK = CK_QD + 16 * FRAG2;
constexpr long CK_KD = CK_QK + 8 * FRAG2;
constexpr long CK_U = CK_KD + 16 * FRAG2;
constexpr long CK_ECL = CK_U + CK_C * CK_D;
constexpr long CK_REC = CK_ECL + 64;
static_assert((CK_REC * 4) % 256 == 0, "records stay 256-byte aligned");

// a double moved by DPP (both halves); lanes without a source, or in rows
// outside ROW_MASK, read 0.0
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_d(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b), CTRL, ROW_MASK, 0xF, true);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), CTRL, ROW_MASK, 0xF, true);
  return __builtin_bit_cast(double, (static_cast<unsigned long long>(static_cast<unsigned>(hi)) << 32) |
                                        static_cast<unsigned>(lo));
}

// An fp32 MFMA operand as bf16 high and low parts.
struct Frag {
  bf16x8_t hi, lo;
};

__device__ __forceinline__ float bf16_lo_half(unsigned w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi_half(unsigned w) { return __uint_as_float(w & 0xffff0000u); }

// x = hi + lo: hi rounds x to bf16, lo rounds the (exact) remainder
__device__ __forceinline__ void split2(float a, float b, unsigned& h, unsigned& l) {
  h = pack_bf16x2(a, b);
  l = pack_bf16x2(a - bf16_lo_half(h), b - bf16_hi_half(h));
}

__device__ __forceinline__ Frag split8(const float (&x)[8]) {
  u32x4_t h, l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    unsigned hh, ll;
    split2(x[2 * i], x[2 * i + 1], hh, ll);
    h[i] = hh;
    l[i] = ll;
  }
  return Frag{__builtin_bit_cast(bf16x8_t, h), __builtin_bit_cast(bf16x8_t, l)};
}

// c + a b over one k-step, the small terms first
__device__ __forceinline__ f32x4_t mfma3(const Frag& a, const Frag& b, f32x4_t c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, c, 0, 0, 0);
}

// lane's operand from a record fragment pair
__device__ __forceinline__ Frag ld_frag(const float* pair, int lane) {
  const char* p = reinterpret_cast<const char*>(pair) + lane * 16;
  return Frag{*reinterpret_cast<const bf16x8_t*>(p), *reinterpret_cast<const bf16x8_t*>(p + 1024)};
}

// the lane's 8 elements of a fragment pair, from fp32 values
__device__ __forceinline__ void st_frag8(float* pair, int lane, const float (&x)[8]) {
  const Frag f = split8(x);
  char* p = reinterpret_cast<char*>(pair) + lane * 16;
  *reinterpret_cast<bf16x8_t*>(p) = f.hi;
  *reinterpret_cast<bf16x8_t*>(p + 1024) = f.lo;
}

// 4 of a lane's 8 elements (e0 .. e0 + 3, e0 = 0 or 4) of a fragment pair
__device__ __forceinline__ void st_frag4(float* pair, int lane, int e0, float a, float b, float c, float d) {
  unsigned h0, l0, h1, l1;
  split2(a, b, h0, l0);
  split2(c, d, h1, l1);
  char* p = reinterpret_cast<char*>(pair) + lane * 16 + e0 * 2;
  *reinterpret_cast<u32x2_t*>(p) = u32x2_t{h0, h1};
  *reinterpret_cast<u32x2_t*>(p + 1024) = u32x2_t{l0, l1};
}

// A result tile's lane holds rows 4 g + v (v < 4) of column r16; when the rows
// are the k index of a fragment pair whose k-step starts at row 32 s of the
// result's block b (rows 16 b ..), its 4 values are elements e0 .. e0 + 3 of
// lane r16 + 16 g' of fragment step s = b / 2
__device__ __forceinline__ void frag_slot(int blk, int g4, int& lane_g, int& e0) {
  lane_g = 2 * (blk & 1) + (g4 >> 1);
  e0 = 4 * (g4 & 1);
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

// eight consecutive activations loaded raw (get() converts them), so that a
// run of loads can be issued before any conversion waits on one of them
template <typename T> struct Raw8;
template <> struct Raw8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ __forceinline__ void get(float* o) const {
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
};
template <> struct Raw8<bf16_t> {
  uint4 u;
  __device__ __forceinline__ void load(const bf16_t* p) { u = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void get(float* o) const {
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = bf16_to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
      o[2 * i + 1] = bf16_to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
  }
};

// lower 16x16 tiles (I, J), J <= I, numbered (0,0) (1,0) (1,1) (2,0) ... (3,3)
__device__ __forceinline__ void tile_ij(int t, int& I, int& J) {
  I = t < 1 ? 0 : t < 3 ? 1 : t < 6 ? 2 : 3;
  J = t - I * (I + 1) / 2;
}

// a lane's operand from a [row][k] bf16 hi / lo LDS tile pair (row stride
// CK_HS): row `row`, k = 32 s + 8 g4 .. + 7
constexpr int CK_HS = CK_D + 8;   // bf16 row stride of the [token][dim] tiles
__device__ __forceinline__ Frag tile_frag(const uint16_t* hi, const uint16_t* lo, int row, int s, int g4) {
  const int o = row * CK_HS + 32 * s + 8 * g4;
  return Frag{*reinterpret_cast<const bf16x8_t*>(hi + o), *reinterpret_cast<const bf16x8_t*>(lo + o)};
}

// 16x16 tile of X Y^T over the 128 dims from split [token][dim] tiles:
// rows xr + l%16 of X and yr + l%16 of Y
__device__ __forceinline__ f32x4_t gram16(const uint16_t* xh, const uint16_t* xl, int xr, const uint16_t* yh,
                                          const uint16_t* yl, int yr, int g4) {
  // every operand read before the first product, so that the reads' LDS
  // latencies overlap instead of each product waiting on its own
  Frag a[4], b[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    a[s] = tile_frag(xh, xl, xr, s, g4);
    b[s] = tile_frag(yh, yl, yr, s, g4);
  }
  __builtin_amdgcn_sched_barrier(0);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma3(a[s], b[s], acc);
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

struct alignas(16) PrepShared {
  union {
    struct {
      uint16_t h[CK_C * CK_HS], l[CK_C * CK_HS];   // normalised q * d^-1/2, split
    } q;
    float Tm[CK_C][CK_LT];     // (I + L)^-1, lower: after the q k^T tiles are done with q
  } u;
  float L[CK_C][CK_LT];        // (k beta k^T) * decay, strictly lower (formed beside the q k^T tiles)
  uint16_t kh[CK_C * CK_HS], kl[CK_C * CK_HS];     // normalised k, split
  float kT[CK_D][CK_LT];       // normalised k, [dim][token]
  float vT[CK_D][CK_LT];       // v * beta, [dim][token]
  float cum[CK_C], beta[CK_C], ecum[CK_C], bec[CK_C], kds[CK_C];
};

template <typename T>
__global__ __launch_bounds__(CK_NT) void dn_chunk_prep_kernel(ChunkPrepArgs<T> A) {
  __shared__ PrepShared sh;
  QM_PHASE_DECL
  QM_PHASE(0);
  // A.parts workgroups per chunk: each forms L and T, then writes its share
  // (all of it, or a quarter) of the record. The parts of a chunk read the
  // same q, k and v rows: consecutive workgroups in this order run on one die
  // (xcd_remap), so the rows come from memory once per chunk, not per part
  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int part = wg % A.parts;
  const int c = (wg / A.parts) % A.n_chunks;
  const int bh = wg / A.parts / A.n_chunks;
  const int span = CK_PARTS / A.parts;       // quarters this workgroup writes
  const int h = bh % A.heads, b = bh / A.heads;
  const int t0 = c * CK_C;
  const int n_valid = min(CK_C, A.seq - t0);
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int g4 = lane >> 4, r16 = lane & 15;
  float* rec = A.ws + ((long)bh * A.n_chunks + c) * CK_REC;
  const int span_sh = span == 1 ? 0 : 2;     // span is 1 or 4
  auto mine = [&](int quarter) __attribute__((always_inline)) { return (quarter >> span_sh) == part; };

  // q, k, v rows: four threads per token, 32 dims each as four runs of 8
  const int t = tid >> 2, p = tid & 3;
  const bool tok_ok = t < n_valid;
  float qn[32];
  {
    // every load at once, the gates first (the cumulative decay is the
    // longest chain); indices are clamped so that no load sits in a branch
    const bool ok = lane < n_valid;
    const long gi = ((long)b * A.seq + t0 + (ok ? lane : 0)) * A.heads + h;
    const float g_raw = A.g[gi], b_raw = A.beta[gi];
    const long tok = (long)b * A.seq + t0 + (tok_ok ? t : 0);
    const float bv_raw = A.beta[tok * A.heads + h];
    const long qo = tok * A.q_stride + (long)(h % A.hk) * CK_D;
    const long vo = tok * A.v_stride + (long)h * CK_D;
    Raw8<T> xq[4], xk[4], xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 8 * (p + 4 * j);
      xq[j].load(A.q + qo + d);
      xk[j].load(A.k + qo + d);
      xv[j].load(A.v + vo + d);
    }
    __builtin_amdgcn_sched_barrier(0);
    float kv[32], vv[32];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xq[j].get(qn + 8 * j);
      xk[j].get(kv + 8 * j);
      xv[j].get(vv + 8 * j);
    }
    const float bv = tok_ok ? bv_raw : 0.f;

    // gates; padding tokens carry g = 0 and beta = 0
    if (wid == 0) {
      const float gv = ok ? g_raw : 0.f;
      const float bl = ok ? b_raw : 0.f;
      // inclusive scan over the 64 lanes in double on DPP (no LDS round
      // trips): row shifts by 1, 2, 4, 8, then lane 15 of each row to the
      // next row (rows 1, 3), then lane 31 to rows 2 and 3
      double s = gv;
      s += dpp_d<0x111, 0xF>(s);
      s += dpp_d<0x112, 0xF>(s);
      s += dpp_d<0x114, 0xF>(s);
      s += dpp_d<0x118, 0xF>(s);
      s += dpp_d<0x142, 0xA>(s);
      s += dpp_d<0x143, 0xC>(s);
      const float cum = static_cast<float>(s);
      const float last = readlane_f(cum, 63);
      const float ec = expf(cum);
      sh.cum[lane] = cum;
      sh.beta[lane] = bl;
      sh.ecum[lane] = ec;
      sh.bec[lane] = bl * ec;
      sh.kds[lane] = expf(last - cum);
      if (lane == 0 && part == 0) rec[CK_ECL] = expf(last);
    }

    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      sq = fmaf(qn[i], qn[i], sq);
      sk = fmaf(kv[i], kv[i], sk);
    }
    sq += dpp_f<0xB1>(sq);    // lane ^ 1
    sk += dpp_f<0xB1>(sk);
    sq += dpp_f<0x4E>(sq);    // lane ^ 2
    sk += dpp_f<0x4E>(sk);
    const float rq = tok_ok ? rsqrt_rn(sq + 1e-6f) : 0.f;
    const float rk = tok_ok ? rsqrt_rn(sk + 1e-6f) : 0.f;
    const float qscale = 0.08838834764831845f;  // 128^-1/2
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      qn[i] = mul_rn(mul_rn(qn[i], rq), qscale);
      kv[i] = mul_rn(kv[i], rk);
      vv[i] = vv[i] * bv;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 8 * (p + 4 * j);
      float xq[8], xk[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) { xq[e] = qn[8 * j + e]; xk[e] = kv[8 * j + e]; }
      const Frag fq = split8(xq), fk = split8(xk);
      *reinterpret_cast<bf16x8_t*>(&sh.u.q.h[t * CK_HS + d]) = fq.hi;
      *reinterpret_cast<bf16x8_t*>(&sh.u.q.l[t * CK_HS + d]) = fq.lo;
      *reinterpret_cast<bf16x8_t*>(&sh.kh[t * CK_HS + d]) = fk.hi;
      *reinterpret_cast<bf16x8_t*>(&sh.kl[t * CK_HS + d]) = fk.lo;
      // the [dim][token] copies only where this workgroup reads them: dims
      // 32 j .. 32 j + 31 of k for its k_dec quarter (j == part) and, with
      // parts, the w columns of parts 0-1 (k dims 64 part ..) and the u
      // columns of parts 2-3 (v dims 64 (part - 2) ..); uniform per j
      const bool all = A.parts == 1;
      if (all || j == part || (part < 2 && j / 2 == part)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sh.kT[d + e][t] = kv[8 * j + e];
      }
      if (all || (part >= 2 && j / 2 == part - 2)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sh.vT[d + e][t] = vv[8 * j + e];
      }
    }
  }
  QM_PHASE(1);
  __syncthreads();
  QM_PHASE(2);

  // q e^cum fragments (QD: token block t / 16, dk step j) from the thread's
  // own q values: its run j of 8 dims is lane t % 16 + 16 p of fragment j
  if (mine(t >> 4)) {
    const float e = sh.ecum[t];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = qn[8 * j + i] * e;
      st_frag8(rec + CK_QD + ((t >> 4) * 4 + j) * FRAG2, (t & 15) + 16 * p, x);
    }
  }
  QM_PHASE(10);
  // qk = (q k^T) * exp(cum_i - cum_j) for j <= i, as QK fragments: tile
  // (I, J) is computed as k_J q_I^T, so that a lane holds 4 consecutive j of
  // one i; tiles 10 and 11 are the zero blocks (0, 1) and (2, 3) above the
  // diagonal that the scan's 32-wide k-steps read. Tile ti belongs to quarter
  // ti % 4; this workgroup's tiles go round-robin to its waves
  {
    // this workgroup's tiles in order: ti = part, part + 4, part + 8 (one
    // quarter) or all 12; the k-th goes to wave k % 4
    for (int k = wid; k < 3 * span; k += 4) {
      const int ti = span == 1 ? part + 4 * k : k;
      int I, J;
      if (ti < 10) tile_ij(ti, I, J);
      else { I = ti == 10 ? 0 : 2; J = I + 1; }
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      if (ti < 10) acc = gram16(sh.kh, sh.kl, 16 * J + r16, sh.u.q.h, sh.u.q.l, 16 * I + r16, g4);
      // the decays' operands are read before any exponential, outside the
      // masks, so that their LDS latencies overlap
      const int i = 16 * I + r16;
      const float ci = sh.cum[i];
      const float4 cj = lds4(&sh.cum[16 * J + 4 * g4]);
      const float cjv[4] = {cj.x, cj.y, cj.z, cj.w};
      float x[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float val = acc[v] * expf(ci - cjv[v]);
        x[v] = ti < 10 && i >= 16 * J + 4 * g4 + v ? val : 0.f;
      }
      int lg, e0;
      frag_slot(J, g4, lg, e0);
      st_frag4(rec + CK_QK + (I * 2 + J / 2) * FRAG2, r16 + 16 * lg, e0, x[0], x[1], x[2], x[3]);
    }
  }
  QM_PHASE(3);
  // L has its own LDS, so its tiles follow the q k^T tiles with no barrier
  // (T takes q's space after the barrier below)
  QM_PHASE(9);

  float (&L)[CK_C][CK_LT] = sh.L;
  float (&Tm)[CK_C][CK_LT] = sh.u.Tm;
  // L = (k k^T) * beta_i * exp(cum_i - cum_j) for j < i
  // three tile slots per wave, all fragments read before the first MFMA.
  // Waves 0-2 take tiles (I, wid) for I = max(wid, 1) .. 3, so that block
  // wid's fragments serve every slot as the B operand; wave 3 takes (3, 3)
  // and (0, 0). Slots past a wave's tiles (wave 2's third, wave 3's third)
  // repeat a tile and store nothing.
  const int wu = __builtin_amdgcn_readfirstlane(wid);
  const int ib = wu < 3 ? max(wu, 1) : 0;
  int tI[3], tJ[3];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    tI[r] = wu < 3 ? min(ib + r, 3) : (r == 0 ? 3 : 0);
    tJ[r] = wu < 3 ? wu : tI[r];
  }
  Frag fb[4], fa[3][4];
#pragma unroll
  for (int st = 0; st < 4; ++st) fb[st] = tile_frag(sh.kh, sh.kl, 16 * tJ[0] + r16, st, g4);
#pragma unroll
  for (int r = 0; r < 3; ++r)
#pragma unroll
    for (int st = 0; st < 4; ++st) fa[r][st] = tile_frag(sh.kh, sh.kl, 16 * tI[r] + r16, st, g4);
  __builtin_amdgcn_sched_barrier(0);
  f32x4_t lacc[3];
#pragma unroll
  for (int r = 0; r < 3; ++r) lacc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int r = 0; r < 3; ++r) {
      // wave 3's (0, 0) tile takes its own block as the B operand
      const Frag& b = (wu == 3 && r > 0) ? fa[r][st] : fb[st];
      lacc[r] = mfma3(fa[r][st], b, lacc[r]);
    }
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    if (wu < 3 ? ib + r > 3 : r == 2) break;
    const int I = tI[r], J = tJ[r];
    const f32x4_t acc = lacc[r];
    const int j = 16 * J + r16;
    const float cj = sh.cum[j];
    const float4 ci = lds4(&sh.cum[16 * I + 4 * g4]), bi = lds4(&sh.beta[16 * I + 4 * g4]);
    const float civ[4] = {ci.x, ci.y, ci.z, ci.w}, biv[4] = {bi.x, bi.y, bi.z, bi.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 16 * I + 4 * g4 + v;
      const float val = (acc[v] * biv[v]) * expf(civ[v] - cj);
      L[i][j] = i > j ? val : 0.f;
    }
  }
  QM_PHASE(4);
  __syncthreads();

  if (wid == 0) {
    // (I + L_II)^-1 for the four diagonal blocks; lane = (block, column):
    // x_i = [i == col] - sum_{k<i} L_ik x_k
    // the block's lower triangle is read first (rows in runs of 4, the
    // zeros above the diagonal included), so that the substitution's
    // dependent chain waits on no LDS read
    const int I = g4, col = r16;
    float4 lr[15][4];
#pragma unroll
    for (int i = 1; i < 16; ++i)
#pragma unroll
      for (int k4 = 0; k4 < (i + 3) / 4; ++k4) lr[i - 1][k4] = lds4(&L[16 * I + i][16 * I + 4 * k4]);
    __builtin_amdgcn_sched_barrier(0);
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = i == col ? 1.f : 0.f;
#pragma unroll
      for (int kk = 0; kk < i; ++kk) {
        const float4 v = lr[i - 1][kk / 4];
        const float l = kk % 4 == 0 ? v.x : kk % 4 == 1 ? v.y : kk % 4 == 2 ? v.z : v.w;
        acc = fmaf(-l, x[kk], acc);
      }
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Tm[16 * I + i][16 * I + col] = x[i];
  } else {
    // the zero blocks (0, 1) and (2, 3) of T, which the 32-wide k-steps of
    // the w and u products read
    for (int idx = tid - 64; idx < 2 * 256; idx += CK_NT - 64) {
      const int blk = idx >> 8, r = (idx >> 4) & 15, cc = idx & 15;
      Tm[32 * blk + r][32 * blk + 16 + cc] = 0.f;
    }
    // k_dec fragments (KD: dk blocks 2 quarter, 2 quarter + 1, token steps
    // 0..1): lane (dk 16 D + r16, tokens 32 s + 8 g4 ..); this workgroup's
    // fragments are f0 .. f0 + 4 span, the i-th to wave 1 + i % 3
    const int f0 = 4 * span * part;
    for (int i = wid - 1; i < 4 * span; i += 3) {
      const int f = f0 + i;
      const int D = f >> 1, s = f & 1;
      const int c0 = 32 * s + 8 * g4;
      const float* row = &sh.kT[16 * D + r16][0];
      const float4 x0 = lds4(row + c0), x1 = lds4(row + c0 + 4);
      float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= sh.kds[c0 + e];
      st_frag8(rec + CK_KD + f * FRAG2, lane, x);
    }
  }
  QM_PHASE(5);
  __syncthreads();

  QM_PHASE(6);
  // blocks of T below the diagonal, one sub-diagonal at a time:
  // T_IJ = -T_II sum_{K=J}^{I-1} L_IK T_KJ
  for (int dist = 1; dist < 4; ++dist) {
    if (wid < 4 - dist) {
      const int J = wid, I = wid + dist;
      f32x4_t pp = {0.f, 0.f, 0.f, 0.f};
      for (int K = J; K < I; ++K) {
        const float4 a = lds4(&L[16 * I + r16][16 * K + 4 * g4]);
        const float* tb = &Tm[16 * K + 4 * g4][16 * J + r16];
        pp = mfma4x4(a, make_float4(tb[0], tb[CK_LT], tb[2 * CK_LT], tb[3 * CK_LT]), pp);
      }
      const float4 xa = lds4(&Tm[16 * I + r16][16 * I + 4 * g4]);
      f32x4_t x = {0.f, 0.f, 0.f, 0.f};
      x = mfma4x4(xa, make_float4(pp[0], pp[1], pp[2], pp[3]), x);
#pragma unroll
      for (int v = 0; v < 4; ++v) Tm[16 * I + 4 * g4 + v][16 * J + r16] = -x[v];
    }
    __syncthreads();
  }

  QM_PHASE(7);
  // w = T (k beta e^cum) and u = T (v beta), as w^T = (k beta e^cum)^T T^T so
  // that a lane holds 4 consecutive dims of one token: quarter r holds column
  // tiles 4 r .. 4 r + 3 of the 16 (w: 0..7, u: 8..15, 16 dims each), one per
  // wave; T is lower triangular, so row block I needs k-steps 0 .. I / 2
  for (int qr = span * part; qr < span * (part + 1); ++qr) {
    const int tile = 4 * qr + wid;
    const bool is_u = tile >= 8;
    const int D = tile & 7;
    const float* arow = is_u ? &sh.vT[16 * D + r16][0] : &sh.kT[16 * D + r16][0];
    // every LDS read first (the A row and its scales, the T rows of the four
    // row blocks), then the splits and products
    float4 ar[2][2], sc[2][2], tr[4][2][2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int c = 32 * s2 + 8 * g4;
      ar[s2][0] = lds4(arow + c);
      ar[s2][1] = lds4(arow + c + 4);
      sc[s2][0] = lds4(&sh.bec[c]);
      sc[s2][1] = lds4(&sh.bec[c + 4]);
    }
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int s2 = 0; s2 <= I / 2; ++s2) {
        const int c = 32 * s2 + 8 * g4;
        tr[I][s2][0] = lds4(&Tm[16 * I + r16][c]);
        tr[I][s2][1] = lds4(&Tm[16 * I + r16][c + 4]);
      }
    __builtin_amdgcn_sched_barrier(0);
    Frag a[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      float x[8] = {ar[s2][0].x, ar[s2][0].y, ar[s2][0].z, ar[s2][0].w,
                    ar[s2][1].x, ar[s2][1].y, ar[s2][1].z, ar[s2][1].w};
      const float y[8] = {sc[s2][0].x, sc[s2][0].y, sc[s2][0].z, sc[s2][0].w,
                          sc[s2][1].x, sc[s2][1].y, sc[s2][1].z, sc[s2][1].w};
      if (!is_u)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= y[e];
      a[s2] = split8(x);
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 <= I / 2; ++s2) {
        const float x[8] = {tr[I][s2][0].x, tr[I][s2][0].y, tr[I][s2][0].z, tr[I][s2][0].w,
                            tr[I][s2][1].x, tr[I][s2][1].y, tr[I][s2][1].z, tr[I][s2][1].w};
        acc = mfma3(a[s2], split8(x), acc);
      }
      // acc[v]: dim 16 D + 4 g4 + v of token 16 I + r16
      if (is_u) {
        *reinterpret_cast<float4*>(rec + CK_U + (16 * I + r16) * CK_D + 16 * D + 4 * g4) =
            make_float4(acc[0], acc[1], acc[2], acc[3]);
      } else {
        int lg, e0;
        frag_slot(D, g4, lg, e0);
        st_frag4(rec + CK_W + (I * 4 + D / 2) * FRAG2, r16 + 16 * lg, e0, acc[0], acc[1], acc[2], acc[3]);
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

// A wave's record operands of one chunk, none of which depends on the
// state: the W and QD fragments of its token block (dk steps 0..3), the QK
// fragments of its token block (j steps 0..1), the KD fragments of its two dk
// blocks (token steps 0..1), its 4 values of u and e^cum_last.
struct ScanOps {
  Frag w[4], qd[4], qk[2], kd[2][2];
  float4 u;
  float ecl;
};

__device__ __forceinline__ void load_scan_ops(const float* rec, int wid, int lane, int r16, int g4, int col0,
                                              ScanOps& o) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    o.w[s] = ld_frag(rec + CK_W + (wid * 4 + s) * FRAG2, lane);
    o.qd[s] = ld_frag(rec + CK_QD + (wid * 4 + s) * FRAG2, lane);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) o.qk[s] = ld_frag(rec + CK_QK + (wid * 2 + s) * FRAG2, lane);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int s = 0; s < 2; ++s) o.kd[t][s] = ld_frag(rec + CK_KD + ((2 * wid + t) * 2 + s) * FRAG2, lane);
  o.u = *reinterpret_cast<const float4*>(rec + CK_U + (16 * wid + r16) * CK_D + col0 + 4 * g4);
  o.ecl = rec[CK_ECL];
}

constexpr int SC_SS = CK_D + 8;   // bf16 row stride of the state tile [column][dk]
constexpr int SC_SV = CK_C + 8;   // bf16 row stride of the v_new tile [column][token]

// lane's A operand of row r16 of a bf16 hi / lo LDS tile pair, k = 32 s + 8 g4 ..
__device__ __forceinline__ Frag lds_frag(const uint16_t* hi, const uint16_t* lo, int stride, int r16, int s, int g4) {
  const int o = r16 * stride + 32 * s + 8 * g4;
  return Frag{*reinterpret_cast<const bf16x8_t*>(hi + o), *reinterpret_cast<const bf16x8_t*>(lo + o)};
}

// columns c and c + 1 of row `r` of a [column][.] bf16 hi / lo tile pair from
// two split values
__device__ __forceinline__ void put2(uint16_t* hi, uint16_t* lo, int stride, int c, int r, float a, float b) {
  unsigned hh, ll;
  split2(a, b, hh, ll);
  hi[c * stride + r] = static_cast<uint16_t>(hh);
  hi[(c + 1) * stride + r] = static_cast<uint16_t>(hh >> 16);
  lo[c * stride + r] = static_cast<uint16_t>(ll);
  lo[(c + 1) * stride + r] = static_cast<uint16_t>(ll >> 16);
}

template <typename T>
__global__ __launch_bounds__(CK_NT) void dn_chunk_scan_kernel(ChunkScanArgs<T> A) {
  // the state slice S^T [column][dk] and the chunk's v_new^T [column][token],
  // as bf16 high and low parts (the A operands of the transposed products)
  __shared__ __attribute__((aligned(16))) uint16_t sSh[CK_COLS * SC_SS], sSl[CK_COLS * SC_SS];
  __shared__ __attribute__((aligned(16))) uint16_t sVh[CK_COLS * SC_SV], sVl[CK_COLS * SC_SV];
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

  // wave wid keeps dk rows 32 wid .. 32 wid + 31 of the slice as two result
  // tiles of S^T: st[t][i] = S[dk 32 wid + 16 t + r16][column 4 g4 + i]
  float* S = A.state + (long)bh * CK_D * CK_D + col0 + 4 * g4;
  f32x4_t st[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const float4 x = *reinterpret_cast<const float4*>(S + (long)(32 * wid + 16 * t + r16) * CK_D);
    st[t] = f32x4_t{x.x, x.y, x.z, x.w};
  }
  // operands two chunks ahead: three register sets, the loop unrolled by
  // three so that no set is copied while its loads are in flight. The state
  // and the first two chunks' operands are requested together: the state
  // first, so that its wait leaves the operand loads in flight
  ScanOps o0, o1, o2;
  load_scan_ops(recs, wid, lane, r16, g4, col0, o0);
  load_scan_ops(recs + (long)min(1, A.n_chunks - 1) * CK_REC, wid, lane, r16, g4, col0, o1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    put2(sSh, sSl, SC_SS, 4 * g4, 32 * wid + 16 * t + r16, st[t][0], st[t][1]);
    put2(sSh, sSl, SC_SS, 4 * g4 + 2, 32 * wid + 16 * t + r16, st[t][2], st[t][3]);
  }
  QM_PHASE(1);

  auto chunk = [&](int ci, const ScanOps& cur, ScanOps& ahead) {
    // chunk ci + 2's operands fly during this one
    if (ci + 2 < A.n_chunks) load_scan_ops(recs + (long)(ci + 2) * CK_REC, wid, lane, r16, g4, col0, ahead);
    __syncthreads();
    // (w S)^T and (q_dec S)^T for tokens 16 wid ..: rows = columns 4 g4 + i,
    // column = token 16 wid + r16
    f32x4_t aw = {0.f, 0.f, 0.f, 0.f}, ao = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const Frag sa = lds_frag(sSh, sSl, SC_SS, r16, s, g4);
      aw = mfma3(sa, cur.w[s], aw);
      ao = mfma3(sa, cur.qd[s], ao);
    }
    put2(sVh, sVl, SC_SV, 4 * g4, 16 * wid + r16, cur.u.x - aw[0], cur.u.y - aw[1]);
    put2(sVh, sVl, SC_SV, 4 * g4 + 2, 16 * wid + r16, cur.u.z - aw[2], cur.u.w - aw[3]);
    __syncthreads();

    // out^T += v_new^T qk^T over the causal token steps (j <= i: steps 0 ..
    // wid / 2; the record's QK holds zeros above the diagonal)
    const Frag va0 = lds_frag(sVh, sVl, SC_SV, r16, 0, g4), va1 = lds_frag(sVh, sVl, SC_SV, r16, 1, g4);
    ao = mfma3(va0, cur.qk[0], ao);
    if (wid >= 2) ao = mfma3(va1, cur.qk[1], ao);
    const int tok = ci * CK_C + 16 * wid + r16;
    if (tok < A.seq) {
      T* o = A.out + (((long)b * A.seq + tok) * A.heads + h) * CK_D + col0 + 4 * g4;
#pragma unroll
      for (int i = 0; i < 4; ++i) Act<T>::store(o, i, ao[i]);
    }

    // S^T = S^T e^cum_last + v_new^T k_dec on this wave's dk rows (the tile
    // is only read again after the next chunk's first barrier)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4_t acc = {st[t][0] * cur.ecl, st[t][1] * cur.ecl, st[t][2] * cur.ecl, st[t][3] * cur.ecl};
      acc = mfma3(va0, cur.kd[t][0], acc);
      acc = mfma3(va1, cur.kd[t][1], acc);
      st[t] = acc;
      put2(sSh, sSl, SC_SS, 4 * g4, 32 * wid + 16 * t + r16, acc[0], acc[1]);
      put2(sSh, sSl, SC_SS, 4 * g4 + 2, 32 * wid + 16 * t + r16, acc[2], acc[3]);
    }
    if (ci < 12) QM_PHASE(2 + ci);
  };

  // at least one chunk (the host sends no empty sequence here): no zero-trip
  // test for the compiler to sink the first operand loads behind
  int ci = 0;
  do {
    chunk(ci, o0, o2);
    if (ci + 1 < A.n_chunks) chunk(ci + 1, o1, o0);
    if (ci + 2 < A.n_chunks) chunk(ci + 2, o2, o1);
    ci += 3;
  } while (ci < A.n_chunks);

#pragma unroll
  for (int t = 0; t < 2; ++t)
    *reinterpret_cast<float4*>(S + (long)(32 * wid + 16 * t + r16) * CK_D) =
        make_float4(st[t][0], st[t][1], st[t][2], st[t][3]);
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
