// Depthwise causal conv1d over (batch, channels, time): the free functions
// causal_conv1d and causal_conv1d_step of reference/layers.py:133-147.
//
//   full[b, c, :] = [state[b, c, :] | x[b, c, :]]            (K-1 + T columns)
//   out[b, c, t]  = act(sum_{j<K} w[c, j] full[b, c, t + j])  (tap 0 oldest)
//   new_state     = full[:, :, T:]                           (the last K-1 columns)
//
// causal_conv1d is the same with a zero state (padding K-1 on the left).
// Products accumulate in float32 in tap order and round once to the activation
// type, then silu rounds again, as the decode and prefill kernels do.

#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int CONV_NT = 256;
constexpr int CONV_MAX_TAPS = 8;

template <typename T>
struct ConvArgs {
  const T* x; const T* state; const T* w; T* out; T* new_state;
  int batch, channels, seq, taps, activation;
};

// full[b, c, i] for i < K-1 + T
template <typename T>
__device__ __forceinline__ float conv_full(const ConvArgs<T>& A, long row, int i) {
  const int hist = A.taps - 1;
  if (i < hist) return A.state ? Act<T>::load(A.state, row * hist + i) : 0.f;
  return Act<T>::load(A.x, row * A.seq + (i - hist));
}

// one thread per output (b, c, t), t fastest: a wave reads consecutive time steps
template <typename T>
__global__ __launch_bounds__(CONV_NT) void conv1d_kernel(ConvArgs<T> A) {
  const long i = (long)blockIdx.x * CONV_NT + threadIdx.x;
  const long n = (long)A.batch * A.channels * A.seq;
  if (i >= n) return;
  const int t = (int)(i % A.seq);
  const long row = i / A.seq;                 // b * channels + c
  const int c = (int)(row % A.channels);
  float v[CONV_MAX_TAPS], w[CONV_MAX_TAPS];
#pragma unroll
  for (int j = 0; j < CONV_MAX_TAPS; ++j)
    if (j < A.taps) {
      v[j] = conv_full(A, row, t + j);
      w[j] = Act<T>::load(A.w, (long)c * A.taps + j);
    }
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < CONV_MAX_TAPS; ++j)
    if (j < A.taps) acc = fmaf(w[j], v[j], acc);
  float y = Act<T>::round(acc);
  if (A.activation) y = Act<T>::round(silu_f(y));
  Act<T>::store(A.out, i, y);
}

// one thread per (b, c) row: the last K-1 columns of full, all read before any
// is written (new_state may be the state itself)
template <typename T>
__global__ __launch_bounds__(CONV_NT) void conv1d_state_kernel(ConvArgs<T> A) {
  const long row = (long)blockIdx.x * CONV_NT + threadIdx.x;
  if (row >= (long)A.batch * A.channels) return;
  const int hist = A.taps - 1;
  float v[CONV_MAX_TAPS];
#pragma unroll
  for (int j = 0; j < CONV_MAX_TAPS - 1; ++j)
    if (j < hist) v[j] = conv_full(A, row, A.seq + j);
#pragma unroll
  for (int j = 0; j < CONV_MAX_TAPS - 1; ++j)
    if (j < hist) Act<T>::store(A.new_state, row * hist + j, v[j]);
}

template <typename T>
int launch_conv(int batch, int channels, int seq, int taps, const void* x, const void* state, const void* weight,
                int activation, void* out, void* new_state, hipStream_t stream) {
  ConvArgs<T> A;
  A.x = static_cast<const T*>(x); A.state = static_cast<const T*>(state); A.w = static_cast<const T*>(weight);
  A.out = static_cast<T*>(out); A.new_state = static_cast<T*>(new_state);
  A.batch = batch; A.channels = channels; A.seq = seq; A.taps = taps; A.activation = activation;
  const long n = (long)batch * channels * seq;
  if (n > 0) {
    hipLaunchKernelGGL(conv1d_kernel<T>, dim3((unsigned)((n + CONV_NT - 1) / CONV_NT)), dim3(CONV_NT), 0, stream, A);
    QM_CHECK_LAUNCH();
  }
  if (new_state && taps > 1) {
    const long rows = (long)batch * channels;
    hipLaunchKernelGGL(conv1d_state_kernel<T>, dim3((unsigned)((rows + CONV_NT - 1) / CONV_NT)), dim3(CONV_NT), 0,
                       stream, A);
    QM_CHECK_LAUNCH();
  }
  return QM_OK;
}

}  // namespace

extern "C" int qm_causal_conv1d(int act_dtype, int batch, int channels, int seq, int taps, const void* x,
                                const void* state, const void* weight, int activation, void* out, void* new_state,
                                hipStream_t stream) {
  if (batch <= 0 || channels <= 0 || seq < 0 || taps < 1 || taps > CONV_MAX_TAPS)
    return qm_fail(QM_ERR_ARG, "qm_causal_conv1d: need batch, channels > 0, seq >= 0 and 1 <= taps <= 8");
  if ((long)batch * channels * seq >= (1l << 31) * CONV_NT)
    return qm_fail(QM_ERR_ARG, "qm_causal_conv1d: too many outputs for one launch");
  if ((seq > 0 && (!x || !out)) || !weight) return qm_fail(QM_ERR_ARG, "qm_causal_conv1d: null pointer");
  if (act_dtype == QM_ACT_F32)
    return launch_conv<float>(batch, channels, seq, taps, x, state, weight, activation, out, new_state, stream);
  if (act_dtype == QM_ACT_BF16)
    return launch_conv<bf16_t>(batch, channels, seq, taps, x, state, weight, activation, out, new_state, stream);
  return qm_fail(QM_ERR_DTYPE, "qm_causal_conv1d: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
}
