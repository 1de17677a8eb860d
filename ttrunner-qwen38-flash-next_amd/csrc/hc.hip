// Hyper-connection read gate and reinjection around each branch, gfx950.
//
// The residual of qwen4exp is `streams` copies of the hidden vector side by side
// (hyper, [M, streams * hidden]). Before a branch, Qwen4ExpModel._gated_residual
// (reference/model.py:53-77) mixes them down to one hidden vector:
//
//   normed = rms_norm(hyper, norm_w) per stream of `hidden`        [M, K]
//   mix    = silu((normed . down^T) / streams)                     [M, rank]
//   gate   = sigmoid(mix . up^T)                                    [M, K]
//   mixed  = mean over streams of gate * normed                    [M, hidden]
//   inject = 2 sigmoid((normed . inject_w^T) / streams)            [M, streams]
//
// and after it _reinject (reference/model.py:79-81) adds the branch output back
// into every stream, scaled by that stream's inject weight.
//
// At decode M is a handful of rows, so both products are streams over the
// weights (down|inject [rank + streams, K], up [K, rank]: about 5 MB each at
// K = 8192, rank 320) and the rest is elementwise. Two launches do the mix:
//
//   hc_norm_down  every workgroup stages its group of up to MG rows of hyper
//                 in LDS, normalises them there (per-stream sums of squares
//                 reduced in a fixed order), and takes R rows of down|inject
//                 against them; the four waves split K into quarters and meet
//                 in LDS. The epilogue applies silu or 2 sigmoid. Workgroup 0
//                 of each row group also writes the normalised rows out.
//   hc_up_mean    a workgroup owns HB hidden positions h and all `streams`
//                 up rows s * hidden + h of them (one contiguous block per
//                 stream), dots them with mix from LDS in 16-byte chunks, sums
//                 each row's chunks in LDS, and finishes the gated mean.
//
// Every rounding the reference makes in the activation dtype is made here at
// the same point (F.linear outputs, the division by streams, silu, sigmoid,
// the gated product, the mean), so bf16 results differ from it only by the
// order of the f32 sums.
#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int HC_NT = 256;
constexpr int HC_MAX_STREAMS = 8;
constexpr int HC_MAX_RANK = 512;
constexpr int HC_LDS = 64 * 1024;   // dynamic LDS of hc_norm_down: MG rows of hyper

template <typename T>
struct HcArgs {
  const T* hyper;      // [M, K]
  const float* norm_w; // [K]
  const T* w_di;       // [n_rows, K]: down rows, then inject rows
  const T* w_up;       // [K, rank]
  T* normed;           // [M, K]
  T* mix;              // [M, rank]
  T* mixed;            // [M, hidden]
  T* inject;           // [M, streams] or null
  int M, streams, hidden, K, rank, n_rows;
  float eps;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float chunk_dot(const uint4& w, const uint4& x, float acc, const bf16_t*) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), __builtin_bit_cast(bf16x2_t, x.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), __builtin_bit_cast(bf16x2_t, x.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), __builtin_bit_cast(bf16x2_t, x.z), acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), __builtin_bit_cast(bf16x2_t, x.w), acc,
                                         false);
}
__device__ __forceinline__ float chunk_dot(const uint4& w, const uint4& x, float acc, const float*) {
  acc = fmaf(__uint_as_float(w.x), __uint_as_float(x.x), acc);
  acc = fmaf(__uint_as_float(w.y), __uint_as_float(x.y), acc);
  acc = fmaf(__uint_as_float(w.z), __uint_as_float(x.z), acc);
  return fmaf(__uint_as_float(w.w), __uint_as_float(x.w), acc);
}

// element i (0..VE-1) of a 16-byte chunk as float, and back
template <typename T> struct Chunk;
template <> struct Chunk<bf16_t> {
  static constexpr int VE = 8;
  __device__ __forceinline__ static float get(const uint4& c, int i) {
    const unsigned w = i < 2 ? c.x : i < 4 ? c.y : i < 6 ? c.z : c.w;
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  }
  __device__ __forceinline__ static uint4 pack(const float* v) {
    uint4 c;
    c.x = f32_to_bf16(v[0]) | (static_cast<unsigned>(f32_to_bf16(v[1])) << 16);
    c.y = f32_to_bf16(v[2]) | (static_cast<unsigned>(f32_to_bf16(v[3])) << 16);
    c.z = f32_to_bf16(v[4]) | (static_cast<unsigned>(f32_to_bf16(v[5])) << 16);
    c.w = f32_to_bf16(v[6]) | (static_cast<unsigned>(f32_to_bf16(v[7])) << 16);
    return c;
  }
};
template <> struct Chunk<float> {
  static constexpr int VE = 4;
  __device__ __forceinline__ static float get(const uint4& c, int i) {
    return __uint_as_float(i == 0 ? c.x : i == 1 ? c.y : i == 2 ? c.z : c.w);
  }
  __device__ __forceinline__ static uint4 pack(const float* v) {
    return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
  }
};

// ---------------------------------------------------------------------------
// normalise + down|inject products. grid (ceil(n_rows / R), ceil(M / MG)).
// Wave w covers columns [w K/4, (w+1) K/4): KQ 16-byte chunks per lane per row.
template <typename T, int MG, int R, int KQ>
__global__ __launch_bounds__(HC_NT) void hc_norm_down_kernel(HcArgs<T> A) {
  constexpr int VE = Chunk<T>::VE;
  extern __shared__ uint4 sx[];                       // [MG][K / VE] chunks
  __shared__ float s_ss[MG * HC_MAX_STREAMS];         // per (row, stream) rsqrt factor
  __shared__ float s_part[4][MG][R];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int K = A.K, CPR = K / VE;                    // chunks per row
  const int QC = CPR / 4;                             // chunks per wave quarter (= 64 KQ)
  const int row0 = blockIdx.x * R, m0 = blockIdx.y * MG;

  // this wave's weights first: R rows x KQ chunks, all in flight
  uint4 wv[R][KQ];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const T* wr = A.w_di + (long)min(row0 + r, A.n_rows - 1) * K + (long)(wid * QC + lane) * VE;
#pragma unroll
    for (int j = 0; j < KQ; ++j) wv[r][j] = *reinterpret_cast<const uint4*>(wr + j * 64 * VE);
  }

  // the norm weights of this thread's chunks (used after the reductions)
  float4 nwv[KQ][VE / 4];
#pragma unroll
  for (int i = 0; i < KQ; ++i)
#pragma unroll
    for (int v = 0; v < VE / 4; ++v)
      nwv[i][v] = reinterpret_cast<const float4*>(A.norm_w + (long)(tid + HC_NT * i) * VE)[v];

  // hyper rows of this group into LDS as stored (rows >= M read row M-1 and are
  // never written out)
#pragma unroll
  for (int m = 0; m < MG; ++m) {
    const T* xr = A.hyper + (long)min(m0 + m, A.M - 1) * K;
#pragma unroll
    for (int i = 0; i < KQ; ++i) {
      const int c = tid + HC_NT * i;
      sx[m * CPR + c] = *reinterpret_cast<const uint4*>(xr + (long)c * VE);
    }
  }
  __syncthreads();

  // sum of squares of each (row, stream): one wave per pair, chunks of the
  // stream in a fixed order, so the result does not depend on scheduling
  const int cps = A.hidden / VE;                      // chunks per stream
  for (int p = wid; p < MG * A.streams; p += 4) {
    const int m = p / A.streams, s = p % A.streams;
    float acc = 0.f;
    for (int c = lane; c < cps; c += 64) {
      const uint4 q = sx[m * CPR + s * cps + c];
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        const float v = Chunk<T>::get(q, i);
        acc = fmaf(v, v, acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) s_ss[m * HC_MAX_STREAMS + s] = rsqrt_rn(add_rn(div_rn(acc, (float)A.hidden), A.eps));
  }
  __syncthreads();

  // normalise in place: bf16((x * r) * w), as rms_norm rounds
#pragma unroll
  for (int i = 0; i < KQ; ++i) {
    const int c = tid + HC_NT * i;
    const int s = (c * VE) / A.hidden;
    float nw[VE];
#pragma unroll
    for (int v = 0; v < VE / 4; ++v) {
      const float4 f = nwv[i][v];
      nw[4 * v] = f.x; nw[4 * v + 1] = f.y; nw[4 * v + 2] = f.z; nw[4 * v + 3] = f.w;
    }
#pragma unroll
    for (int m = 0; m < MG; ++m) {
      const float r = s_ss[m * HC_MAX_STREAMS + s];
      const uint4 q = sx[m * CPR + c];
      float y[VE];
#pragma unroll
      for (int v = 0; v < VE; ++v) y[v] = mul_rn(mul_rn(Chunk<T>::get(q, v), r), nw[v]);
      const uint4 o = Chunk<T>::pack(y);
      sx[m * CPR + c] = o;
      if (blockIdx.x == 0 && m0 + m < A.M)
        *reinterpret_cast<uint4*>(A.normed + (long)(m0 + m) * K + (long)c * VE) = o;
    }
  }
  __syncthreads();

  float acc[MG][R];
#pragma unroll
  for (int m = 0; m < MG; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
#pragma unroll
  for (int j = 0; j < KQ; ++j) {
#pragma unroll
    for (int m = 0; m < MG; ++m) {
      const uint4 xq = sx[m * CPR + wid * QC + j * 64 + lane];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = chunk_dot(wv[r][j], xq, acc[m][r], static_cast<const T*>(nullptr));
    }
  }
#pragma unroll
  for (int m = 0; m < MG; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(acc[m][r]);
      if (lane == 0) s_part[wid][m][r] = v;
    }
  __syncthreads();

  if (tid < MG * R) {
    const int m = tid / R, r = tid % R;
    const int row = row0 + r, mm = m0 + m;
    if (row < A.n_rows && mm < A.M) {
      const float lin = Act<T>::round(((s_part[0][m][r] + s_part[1][m][r]) + s_part[2][m][r]) + s_part[3][m][r]);
      const float t = Act<T>::round(div_rn(lin, (float)A.streams));
      if (row < A.rank) {
        Act<T>::store(A.mix, (long)mm * A.rank + row, silu_f(t));
      } else {
        const float sg = Act<T>::round(sigmoid_f(t));
        Act<T>::store(A.inject, (long)mm * A.streams + (row - A.rank), 2.0f * sg);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// up products, sigmoid and the gated mean. grid (hidden / HB, ceil(M / MG)).
// NQ = ceil(streams * HB * rank / VE / 256) 16-byte chunks per thread.
template <typename T, int MG, int HB, int NQ>
__global__ __launch_bounds__(HC_NT) void hc_up_mean_kernel(HcArgs<T> A) {
  constexpr int VE = Chunk<T>::VE;
  __shared__ uint4 s_mix[MG * HC_MAX_RANK / VE];
  __shared__ float s_gate[MG][HC_MAX_STREAMS][HB];
  extern __shared__ float s_part[];                   // [MG][streams * HB][CK + 1]
  const int tid = threadIdx.x;
  const int h0 = blockIdx.x * HB, m0 = blockIdx.y * MG;
  const int CK = A.rank / VE;                         // chunks per up row
  const int per_stream = HB * CK;
  const int total = A.streams * per_stream;
  const int stride = CK + 1;

  uint4 wq[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = min(tid + HC_NT * i, total - 1);
    const int s = q / per_stream, w = q - s * per_stream;
    const int hr = w / CK, kc = w - hr * CK;
    wq[i] = *reinterpret_cast<const uint4*>(A.w_up + ((long)(s * A.hidden + h0 + hr) * A.rank + kc * VE));
  }
  for (int c = tid; c < MG * CK; c += HC_NT) {
    const int m = c / CK, kc = c - m * CK;
    s_mix[c] = *reinterpret_cast<const uint4*>(A.mix + (long)min(m0 + m, A.M - 1) * A.rank + kc * VE);
  }
  // the normalised value this thread gates later: thread p owns (row m, stream
  // s, position hr), p < MG * streams * HB <= 256
  const int gm = tid / (A.streams * HB), gs = (tid / HB) % A.streams, ghr = tid % HB;
  const float nv = Act<T>::load(A.normed, (long)min(m0 + gm, A.M - 1) * A.K + min(gs * A.hidden + h0 + ghr, A.K - 1));
  __syncthreads();

#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + HC_NT * i;
    if (q < total) {
      const int s = q / per_stream, w = q - s * per_stream;
      const int hr = w / CK, kc = w - hr * CK;
#pragma unroll
      for (int m = 0; m < MG; ++m)
        s_part[(m * A.streams * HB + s * HB + hr) * stride + kc] =
            chunk_dot(wq[i], s_mix[m * CK + kc], 0.f, static_cast<const T*>(nullptr));
    }
  }
  __syncthreads();

  if (tid < MG * A.streams * HB) {
    const float* pr = s_part + (long)tid * stride;
    float lin = 0.f;
    for (int kc = 0; kc < CK; ++kc) lin += pr[kc];
    const float g = Act<T>::round(sigmoid_f(Act<T>::round(lin)));
    s_gate[gm][gs][ghr] = Act<T>::round(g * nv);
  }
  __syncthreads();

  if (tid < MG * HB) {
    const int m = tid / HB, hr = tid % HB;
    if (m0 + m < A.M) {
      float sum = 0.f;
      for (int s = 0; s < A.streams; ++s) sum += s_gate[m][s][hr];
      Act<T>::store(A.mixed, (long)(m0 + m) * A.hidden + h0 + hr, div_rn(sum, (float)A.streams));
    }
  }
}

// ---------------------------------------------------------------------------
// out[m][s*hidden + h] = hyper[m][s*hidden + h] + branch[m][h] * inject[m][s]
// (each product and sum rounded to the activation dtype, never fused, so the
// result is the reference's bit for bit); VE elements a thread.
template <typename T>
__global__ __launch_bounds__(HC_NT) void hc_reinject_kernel(const T* hyper, const T* branch, const T* inject,
                                                             T* out, int M, int streams, int hidden) {
  constexpr int VE = Chunk<T>::VE;
  const long K = (long)streams * hidden;
  const long c = (long)blockIdx.x * HC_NT + threadIdx.x;     // chunk of [M, K]
  if (c >= M * K / VE) return;
  const long e = c * VE;
  const int m = (int)(e / K);
  const long col = e - m * K;
  const int s = (int)(col / hidden), h = (int)(col - (long)s * hidden);
  const float inj = Act<T>::load(inject, (long)m * streams + s);
  const uint4 hq = *reinterpret_cast<const uint4*>(hyper + e);
  const uint4 bq = *reinterpret_cast<const uint4*>(branch + (long)m * hidden + h);
  float y[VE];
#pragma unroll
  for (int v = 0; v < VE; ++v)
    y[v] = add_rn(Chunk<T>::get(hq, v), Act<T>::round(mul_rn(Chunk<T>::get(bq, v), inj)));
  *reinterpret_cast<uint4*>(out + e) = Chunk<T>::pack(y);
}

// ---------------------------------------------------------------------------

struct HcLayout {
  size_t normed, mix, total;
};

HcLayout hc_layout(const qm_hc_geom& g) {
  const size_t es = g.act_dtype == QM_ACT_BF16 ? 2 : 4;
  HcLayout L;
  L.normed = 0;
  L.mix = qm_align256((size_t)g.rows * g.streams * g.hidden * es);
  L.total = L.mix + qm_align256((size_t)g.rows * g.rank * es);
  return L;
}

// R rows of down|inject per wave; hc_up_mean takes MG_UP rows and HB hidden
// positions a workgroup (HB x streams up rows: 5 KB at bf16, rank 320, 4 streams).
// hc_norm_down stages as many rows (MG, at most 4) as fit HC_LDS.
template <typename T> struct HcTile;
template <> struct HcTile<bf16_t> { static constexpr int R = 2, MG_UP = 4, HB = 8; };
template <> struct HcTile<float> { static constexpr int R = 2, MG_UP = 2, HB = 4; };

int hc_up_chunks(const qm_hc_geom& g) {   // 16-byte up chunks of one hc_up_mean workgroup
  return g.act_dtype == QM_ACT_BF16 ? g.streams * HcTile<bf16_t>::HB * (g.rank / 8)
                                    : g.streams * HcTile<float>::HB * (g.rank / 4);
}

// rows of a workgroup's group: the fewest of 1, 2, 4 that cover M (at most
// `cap`, and for hc_norm_down at most what fits HC_LDS)
int hc_group_rows(int M, int cap) {
  const int need = M >= 3 ? 4 : M;
  return need < cap ? need : cap;
}

int hc_down_rows(long K, int es, int M) {
  int mg = 4;
  while (mg > 1 && (long)mg * K * es > HC_LDS) mg /= 2;
  return hc_group_rows(M, mg);
}

bool hc_kq_ok(long kq) { return kq == 1 || kq == 2 || kq == 4 || kq == 5 || kq == 8 || kq == 10; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

const char* hc_check(const qm_hc_geom* g) {
  if (!g) return "qm_hc: null geometry";
  if (g->act_dtype != QM_ACT_BF16 && g->act_dtype != QM_ACT_F32) return "qm_hc: act_dtype must be F32 or BF16";
  if (g->rows <= 0 || g->hidden <= 0 || g->streams <= 0 || g->rank <= 0) return "qm_hc: bad sizes";
  if (g->streams > HC_MAX_STREAMS) return "qm_hc: at most 8 streams";
  const int ve = g->act_dtype == QM_ACT_BF16 ? 8 : 4;
  const long K = (long)g->streams * g->hidden;
  if (g->hidden % 8) return "qm_hc: hidden must be a multiple of 8";
  if (K % (4L * 64 * ve) || !hc_kq_ok(K / (4L * 64 * ve)))
    return "qm_hc: streams * hidden must be 1, 2, 4, 5, 8 or 10 times 2048 (bf16) or 1024 (f32)";
  if (K * (ve == 8 ? 2 : 4) > HC_LDS) return "qm_hc: streams * hidden too wide for LDS staging";
  if (g->rank % ve || g->rank > HC_MAX_RANK) return "qm_hc: rank must be a multiple of 8 (4 for f32), at most 512";
  if (hc_up_chunks(*g) > 8 * HC_NT) return "qm_hc: streams * rank too large";
  return nullptr;
}

template <typename T, int MG, int NQ>
void launch_up_mg(const HcArgs<T>& A, hipStream_t stream) {
  constexpr int HB = HcTile<T>::HB;
  const size_t lds = (size_t)MG * A.streams * HB * (A.rank / Chunk<T>::VE + 1) * sizeof(float);
  hipLaunchKernelGGL((hc_up_mean_kernel<T, MG, HB, NQ>), dim3(A.hidden / HB, (A.M + MG - 1) / MG), dim3(HC_NT), lds,
                     stream, A);
}

template <typename T, int NQ>
void launch_up(const HcArgs<T>& A, hipStream_t stream) {
  const int mg = hc_group_rows(A.M, HcTile<T>::MG_UP);
  if (mg >= 4) launch_up_mg<T, HcTile<T>::MG_UP, NQ>(A, stream);
  else if (mg == 2) launch_up_mg<T, 2, NQ>(A, stream);
  else launch_up_mg<T, 1, NQ>(A, stream);
}

template <typename T, int MG, int KQ>
void launch_down_mg(const HcArgs<T>& A, hipStream_t stream) {
  constexpr int R = HcTile<T>::R;
  const size_t lds = (size_t)MG * A.K * sizeof(T);
  hipLaunchKernelGGL((hc_norm_down_kernel<T, MG, R, KQ>), dim3((A.n_rows + R - 1) / R, (A.M + MG - 1) / MG),
                     dim3(HC_NT), lds, stream, A);
}

template <typename T, int KQ>
void launch_down(const HcArgs<T>& A, hipStream_t stream) {
  const int mg = hc_down_rows(A.K, sizeof(T), A.M);
  if (mg == 4) launch_down_mg<T, 4, KQ>(A, stream);
  else if (mg == 2) launch_down_mg<T, 2, KQ>(A, stream);
  else launch_down_mg<T, 1, KQ>(A, stream);
}

template <typename T>
int run_mix(const qm_hc_geom& g, const void* hyper, const float* norm_w, const void* w_di, int with_inject,
            const void* w_up, void* mixed, void* inject, void* ws, hipStream_t stream) {
  const HcLayout L = hc_layout(g);
  HcArgs<T> A;
  A.hyper = static_cast<const T*>(hyper);
  A.norm_w = norm_w;
  A.w_di = static_cast<const T*>(w_di);
  A.w_up = static_cast<const T*>(w_up);
  A.normed = reinterpret_cast<T*>(static_cast<char*>(ws) + L.normed);
  A.mix = reinterpret_cast<T*>(static_cast<char*>(ws) + L.mix);
  A.mixed = static_cast<T*>(mixed);
  A.inject = static_cast<T*>(inject);
  A.M = g.rows; A.streams = g.streams; A.hidden = g.hidden; A.K = g.streams * g.hidden; A.rank = g.rank;
  A.n_rows = g.rank + (with_inject ? g.streams : 0);
  A.eps = g.eps;
  constexpr int VE = Chunk<T>::VE;
  switch (A.K / (4 * 64 * VE)) {
    case 1: launch_down<T, 1>(A, stream); break;
    case 2: launch_down<T, 2>(A, stream); break;
    case 4: launch_down<T, 4>(A, stream); break;
    case 5: launch_down<T, 5>(A, stream); break;
    case 8: launch_down<T, 8>(A, stream); break;
    case 10: launch_down<T, 10>(A, stream); break;
    default: return qm_fail(QM_ERR_UNSUPPORTED, "qm_hc_mix: unsupported streams * hidden");
  }
  QM_CHECK_LAUNCH();
  const int nq = (hc_up_chunks(g) + HC_NT - 1) / HC_NT;
  switch (nq) {
    case 1: launch_up<T, 1>(A, stream); break;
    case 2: launch_up<T, 2>(A, stream); break;
    case 3: launch_up<T, 3>(A, stream); break;
    case 4: launch_up<T, 4>(A, stream); break;
    case 5: launch_up<T, 5>(A, stream); break;
    case 6: launch_up<T, 6>(A, stream); break;
    case 7: launch_up<T, 7>(A, stream); break;
    case 8: launch_up<T, 8>(A, stream); break;
    default: return qm_fail(QM_ERR_UNSUPPORTED, "qm_hc_mix: streams * rank too large");
  }
  QM_CHECK_LAUNCH();
  return QM_OK;
}

}  // namespace

extern "C" size_t qm_hc_mix_workspace(const qm_hc_geom* g) {
  if (hc_check(g)) return 0;
  return hc_layout(*g).total;
}

extern "C" int qm_hc_mix(const qm_hc_geom* g, const void* hyper, const float* norm_w, const void* down_inject_w,
                         int with_inject, const void* up_w, void* mixed, void* inject, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  if (const char* why = hc_check(g)) return qm_fail(QM_ERR_ARG, why);
  if (!hyper || !norm_w || !down_inject_w || !up_w || !mixed || !workspace)
    return qm_fail(QM_ERR_ARG, "qm_hc_mix: null pointer");
  if (!aligned16(hyper) || !aligned16(norm_w) || !aligned16(down_inject_w) || !aligned16(up_w) ||
      !aligned16(workspace))
    return qm_fail(QM_ERR_ARG, "qm_hc_mix: hyper, weights and workspace must be 16-byte aligned");
  if (with_inject && !inject) return qm_fail(QM_ERR_ARG, "qm_hc_mix: with_inject needs an inject output");
  if (workspace_bytes < hc_layout(*g).total) return qm_fail(QM_ERR_WORKSPACE, "qm_hc_mix: workspace too small");
  if (g->act_dtype == QM_ACT_BF16)
    return run_mix<bf16_t>(*g, hyper, norm_w, down_inject_w, with_inject, up_w, mixed, inject, workspace, stream);
  return run_mix<float>(*g, hyper, norm_w, down_inject_w, with_inject, up_w, mixed, inject, workspace, stream);
}

extern "C" int qm_hc_reinject(const qm_hc_geom* g, const void* hyper, const void* branch, const void* inject,
                              void* out, hipStream_t stream) {
  if (!g) return qm_fail(QM_ERR_ARG, "qm_hc_reinject: null geometry");
  if (g->act_dtype != QM_ACT_BF16 && g->act_dtype != QM_ACT_F32)
    return qm_fail(QM_ERR_DTYPE, "qm_hc_reinject: act_dtype must be F32 or BF16");
  if (g->rows <= 0 || g->streams <= 0 || g->hidden <= 0 || g->hidden % 8)
    return qm_fail(QM_ERR_ARG, "qm_hc_reinject: bad sizes (hidden a multiple of 8)");
  if (!hyper || !branch || !inject || !out) return qm_fail(QM_ERR_ARG, "qm_hc_reinject: null pointer");
  if (!aligned16(hyper) || !aligned16(branch) || !aligned16(out))
    return qm_fail(QM_ERR_ARG, "qm_hc_reinject: hyper, branch and out must be 16-byte aligned");
  const int ve = g->act_dtype == QM_ACT_BF16 ? 8 : 4;
  const long chunks = (long)g->rows * g->streams * g->hidden / ve;
  const dim3 grid((unsigned)((chunks + HC_NT - 1) / HC_NT));
  if (g->act_dtype == QM_ACT_BF16)
    hipLaunchKernelGGL(hc_reinject_kernel<bf16_t>, grid, dim3(HC_NT), 0, stream, static_cast<const bf16_t*>(hyper),
                       static_cast<const bf16_t*>(branch), static_cast<const bf16_t*>(inject),
                       static_cast<bf16_t*>(out), g->rows, g->streams, g->hidden);
  else
    hipLaunchKernelGGL(hc_reinject_kernel<float>, grid, dim3(HC_NT), 0, stream, static_cast<const float*>(hyper),
                       static_cast<const float*>(branch), static_cast<const float*>(inject),
                       static_cast<float*>(out), g->rows, g->streams, g->hidden);
  QM_CHECK_LAUNCH();
  return QM_OK;
}
