// Small-M projections of a layer, gfx950: y[m][n] = sum_k W[n][k] x[m][k].
//
// The layer GEMVs around the token-mixing core (reference/model.py:184-187,
// 244, 270, 274, 345-352, 383) at M <= 4 activation rows are a stream over the
// weights: each weight byte is used M times. The projections that read the
// same input are concatenated row-wise once (qkv | gate | beta | alpha for the
// DeltaNet layer; q | k | v | indexer q | indexer k for the QSA layer), so one
// launch streams them all, and a segment table sends each row range to its own
// output tensor.
//
// qm_gemv_reinject is the output projection of a branch with the
// hyper-connection reinjection (reference/model.py:79-81) as its epilogue:
// each output y[m][j], rounded as F.linear rounds it, is added into every
// stream s of the residual, hyper[m][s * n + j] += round(y * inject[m][s]), so
// the branch output never goes through memory.
//
// Work split: a 256-thread workgroup of four waves; wave w takes R consecutive
// weight rows. A lane owns fixed 16-byte column chunks (8 bf16 or 4 fp32 per
// chunk, chunk c = lane + 64 j), so every wave-wide weight load reads 1 KB of
// contiguous memory, and all R x KC of a wave's loads are issued before the
// first multiply. The M activation rows are staged in LDS once per workgroup,
// as stored. bf16 chunks meet in v_dot2_f32_bf16 (two exact products added in
// f32 per instruction), f32 chunks in FMAs. Each (row, m) partial is summed
// over the wave's lanes at the end.
#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int GV_NT = 256;
constexpr int GV_MAX_M = 4;
constexpr int GV_RJ_PRE = 8;       // reinjection streams whose residual values load with the weights

template <typename T>
struct GemvArgs {
  const T* w;     // [N, K]
  const T* x;     // [M, K]
  int M, N, K;
  int n_seg;
  int seg_end[QM_GEMV_MAX_SEG];
  T* seg_out[QM_GEMV_MAX_SEG];   // rows [seg_end[s-1], seg_end[s]) -> seg_out[s] as [M, rows of s]
  T* hyper;                      // reinjection: [M, streams * N], updated in place
  const T* inject;               //              [M, streams]
  int streams;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// one 16-byte weight chunk against the matching activation chunk, into acc
__device__ __forceinline__ float chunk_dot(const uint4& w, const uint4& x, float acc, const bf16_t*) {
  // v_dot2_f32_bf16: two bf16 products (exact in f32) added to acc in f32
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

template <typename T, int MM, int R, int KC, bool RJ>
__global__ __launch_bounds__(GV_NT) void gemv_kernel(GemvArgs<T> A) {
  constexpr int VE = 16 / sizeof(T);          // elements per 16-byte chunk
  constexpr int CPR = KC * 64;                // 16-byte chunks per row
  extern __shared__ uint4 sx[];               // [MM][CPR] activation chunks, as stored
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int row0 = (blockIdx.x * (GV_NT / 64) + wid) * R;

  // this wave's weights, all loads in flight before any arithmetic
  uint4 wv[R][KC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const T* wr = A.w + (long)min(row0 + r, A.N - 1) * A.K + lane * VE;
#pragma unroll
    for (int j = 0; j < KC; ++j) wv[r][j] = *reinterpret_cast<const uint4*>(wr + j * 64 * VE);
  }
  // reinjection: the residual values and inject weights this lane will update
  // (lane = (row r, activation row m) of the epilogue), in the same round trip
  // as the weights rather than after the reduction; indices clamped
  float hv[GV_RJ_PRE], iv[GV_RJ_PRE];
  if constexpr (RJ) {
    if (lane < R * MM) {
      const int row = min(row0 + lane % R, A.N - 1), mc = min(lane / R, A.M - 1);
#pragma unroll
      for (int s = 0; s < GV_RJ_PRE; ++s) {
        const int sc = min(s, A.streams - 1);
        hv[s] = Act<T>::load(A.hyper, ((long)mc * A.streams + sc) * A.N + row);
        iv[s] = Act<T>::load(A.inject, (long)mc * A.streams + sc);
      }
    }
  }
  // the activation rows, all of a thread's 16-byte loads at once; rows >= M are zero
  constexpr int XC = (MM * CPR + GV_NT - 1) / GV_NT;
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = min(tid + GV_NT * i, A.M * CPR - 1);
    xr[i] = *reinterpret_cast<const uint4*>(A.x + (long)c * VE);
  }
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = tid + GV_NT * i;
    if (c < MM * CPR) sx[c] = c < A.M * CPR ? xr[i] : make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();

  float acc[MM][R];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
#pragma unroll
  for (int j = 0; j < KC; ++j) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const uint4 xq = sx[m * CPR + j * 64 + lane];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = chunk_dot(wv[r][j], xq, acc[m][r], static_cast<const T*>(nullptr));
    }
  }
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = wave_sum(acc[m][r]);

  if (lane < R * MM) {
    const int r = lane % R, m = lane / R;
    const int row = row0 + r;
    float v = 0.f;
#pragma unroll
    for (int mm = 0; mm < MM; ++mm)
#pragma unroll
      for (int rr = 0; rr < R; ++rr) v = (mm == m && rr == r) ? acc[mm][rr] : v;
    if (row < A.N && m < A.M) {
      if constexpr (RJ) {
        const float y = Act<T>::round(v);
#pragma unroll
        for (int s = 0; s < GV_RJ_PRE; ++s)
          if (s < A.streams)
            Act<T>::store(A.hyper, ((long)m * A.streams + s) * A.N + row, add_rn(hv[s], Act<T>::round(mul_rn(y, iv[s]))));
        for (int s = GV_RJ_PRE; s < A.streams; ++s) {
          const long i = ((long)m * A.streams + s) * A.N + row;
          const float inj = Act<T>::load(A.inject, (long)m * A.streams + s);
          Act<T>::store(A.hyper, i, add_rn(Act<T>::load(A.hyper, i), Act<T>::round(mul_rn(y, inj))));
        }
      } else {
        int s = 0, start = 0;
        while (s + 1 < A.n_seg && row >= A.seg_end[s]) { start = A.seg_end[s]; ++s; }
        const int n_s = A.seg_end[s] - start;
        Act<T>::store(A.seg_out[s], (long)m * n_s + (row - start), v);
      }
    }
  }
}

template <typename T, int MM, bool RJ>
int launch_mm(const GemvArgs<T>& A, hipStream_t stream) {
  constexpr int VE = 16 / sizeof(T);
  const int kc = A.K / (64 * VE);
  const size_t lds = (size_t)MM * A.K * sizeof(T);
  // one row of KC chunks of 1 KB in flight per wave (4 KB at k = 2048, 8 KB at
  // k = 4096, bf16): more workgroups with fewer rows each measured faster than
  // 16 KB per wave. A 48-layer step went 1707 -> 1696 us (one row at k = 4096:
  // 512 workgroups for an output projection), -> 1666 us (two rows at k =
  // 2048), -> 1653 us (one row: 3088 workgroups for the DeltaNet input
  // projection)
  if (kc == 4) {
    const int rows = (GV_NT / 64) * 1;
    hipLaunchKernelGGL((gemv_kernel<T, MM, 1, 4, RJ>), dim3((A.N + rows - 1) / rows), dim3(GV_NT), lds, stream, A);
  } else if (kc == 8) {
    const int rows = (GV_NT / 64) * 1;
    hipLaunchKernelGGL((gemv_kernel<T, MM, 1, 8, RJ>), dim3((A.N + rows - 1) / rows), dim3(GV_NT), lds, stream, A);
  } else if (kc == 16) {
    const int rows = (GV_NT / 64) * 1;
    hipLaunchKernelGGL((gemv_kernel<T, MM, 1, 16, RJ>), dim3((A.N + rows - 1) / rows), dim3(GV_NT), lds, stream, A);
  } else {
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_gemv: k must be 2048 or 4096 (bf16), 1024, 2048 or 4096 (f32)");
  }
  QM_CHECK_LAUNCH();
  return QM_OK;
}

template <typename T, bool RJ>
int launch_m(const GemvArgs<T>& A, hipStream_t stream) {
  switch (A.M) {
    case 1: return launch_mm<T, 1, RJ>(A, stream);
    case 2: return launch_mm<T, 2, RJ>(A, stream);
    default: return launch_mm<T, 4, RJ>(A, stream);
  }
}

template <typename T>
int launch_gemv(int m, int n, int k, const void* w, const void* x, int n_seg, const int* seg_rows,
                void* const* seg_out, hipStream_t stream) {
  GemvArgs<T> A = {};
  A.w = static_cast<const T*>(w); A.x = static_cast<const T*>(x);
  A.M = m; A.N = n; A.K = k; A.n_seg = n_seg;
  int end = 0;
  for (int s = 0; s < n_seg; ++s) {
    end += seg_rows[s];
    A.seg_end[s] = end;
    A.seg_out[s] = static_cast<T*>(seg_out[s]);
  }
  if (end != n) return qm_fail(QM_ERR_ARG, "qm_gemv: segment rows must add up to n");
  return launch_m<T, false>(A, stream);
}

template <typename T>
int launch_reinject(int m, int n, int k, const void* w, const void* x, int streams, const void* inject, void* hyper,
                    hipStream_t stream) {
  GemvArgs<T> A = {};
  A.w = static_cast<const T*>(w); A.x = static_cast<const T*>(x);
  A.M = m; A.N = n; A.K = k; A.n_seg = 1; A.seg_end[0] = n;
  A.hyper = static_cast<T*>(hyper); A.inject = static_cast<const T*>(inject); A.streams = streams;
  return launch_m<T, true>(A, stream);
}

}  // namespace

extern "C" int qm_gemv(int act_dtype, int m, int n, int k, const void* w, const void* x, int n_seg,
                       const int* seg_rows, void* const* seg_out, hipStream_t stream) {
  if (m <= 0 || m > GV_MAX_M) return qm_fail(QM_ERR_UNSUPPORTED, "qm_gemv: m must be 1..4");
  if (n <= 0 || k <= 0) return qm_fail(QM_ERR_ARG, "qm_gemv: bad sizes");
  if (!w || !x || !seg_rows || !seg_out) return qm_fail(QM_ERR_ARG, "qm_gemv: null pointer");
  if (n_seg <= 0 || n_seg > QM_GEMV_MAX_SEG) return qm_fail(QM_ERR_ARG, "qm_gemv: 1..8 output segments");
  for (int s = 0; s < n_seg; ++s)
    if (seg_rows[s] <= 0 || !seg_out[s]) return qm_fail(QM_ERR_ARG, "qm_gemv: empty segment or null output");
  const bool k_ok = act_dtype == QM_ACT_BF16 ? (k == 2048 || k == 4096) : (k == 1024 || k == 2048 || k == 4096);
  if (!k_ok) return qm_fail(QM_ERR_UNSUPPORTED, "qm_gemv: k must be 2048 or 4096 (bf16), 1024, 2048 or 4096 (f32)");
  if (act_dtype == QM_ACT_BF16) return launch_gemv<bf16_t>(m, n, k, w, x, n_seg, seg_rows, seg_out, stream);
  if (act_dtype == QM_ACT_F32) return launch_gemv<float>(m, n, k, w, x, n_seg, seg_rows, seg_out, stream);
  return qm_fail(QM_ERR_DTYPE, "qm_gemv: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
}

extern "C" int qm_gemv_reinject(int act_dtype, int m, int n, int k, const void* w, const void* x, int streams,
                                const void* inject, void* hyper, hipStream_t stream) {
  if (m <= 0 || m > GV_MAX_M) return qm_fail(QM_ERR_UNSUPPORTED, "qm_gemv_reinject: m must be 1..4");
  if (n <= 0 || k <= 0 || streams <= 0) return qm_fail(QM_ERR_ARG, "qm_gemv_reinject: bad sizes");
  if (!w || !x || !inject || !hyper) return qm_fail(QM_ERR_ARG, "qm_gemv_reinject: null pointer");
  const bool k_ok = act_dtype == QM_ACT_BF16 ? (k == 2048 || k == 4096) : (k == 1024 || k == 2048 || k == 4096);
  if (!k_ok)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_gemv_reinject: k must be 2048 or 4096 (bf16), 1024, 2048 or 4096 (f32)");
  if (act_dtype == QM_ACT_BF16) return launch_reinject<bf16_t>(m, n, k, w, x, streams, inject, hyper, stream);
  if (act_dtype == QM_ACT_F32) return launch_reinject<float>(m, n, k, w, x, streams, inject, hyper, stream);
  return qm_fail(QM_ERR_DTYPE, "qm_gemv_reinject: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
}
