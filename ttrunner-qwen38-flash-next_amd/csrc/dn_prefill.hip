// Gated DeltaNet over a chunk of S tokens (prefill), gfx950.
//
// The seq > 1 body of Qwen4ExpModel._linear_attention (reference/model.py:
// 198-201, 205-217, 230-243): the causal conv over [history | chunk] with the
// last K-1 inputs carried to the ring, the gates, the delta rule over the chunk,
// and the gated RMS norm. Launches:
//   dn_conv_chunk   one thread per (sequence, channel): slides the K-tap window
//                   down the chunk in registers, then writes the ring; the same
//                   grid computes beta and g for every (token, head)
//   delta rule      qm_dn_chunk_wy (WY/UT chunked form) when the chunk fills
//                   64-token sub-chunks, else the token loop
//   dn_gated_norm   one wavefront per (token, head) row of 128
#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int DN_D = 128;

template <typename T>
struct ConvChunkArgs {
  const T* qkv; const T* a; const T* b; const float* a_neg; const float* dt_bias; const T* conv_w;
  const int* positions; T* ring; T* conv_out; float* g_out; float* beta_out;
  int batch, seq, conv_dim, K, hv;
};

template <typename T>
__global__ __launch_bounds__(256) void dn_conv_chunk_kernel(ConvChunkArgs<T> A) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long n_conv = (long)A.batch * A.conv_dim;
  if (gid < n_conv) {
    const int b = gid / A.conv_dim, ch = gid % A.conv_dim;
    const int K = A.K;
    const int pos0 = A.positions[b];
    T* ring = A.ring + ((long)b * A.conv_dim + ch) * K;
    float w[8], win[8];
    for (int j = 0; j < K; ++j) w[j] = Act<T>::load(A.conv_w, (long)ch * K + j);
    // win[0..K-2] = inputs of positions pos0-K+1 .. pos0-1 (oldest first)
    for (int j = 0; j < K - 1; ++j) {
      int slot = (pos0 - (K - 1) + j) % K;
      if (slot < 0) slot += K;
      win[j] = Act<T>::load(ring, slot);
    }
    for (int t = 0; t < A.seq; ++t) {
      const long idx = ((long)b * A.seq + t) * A.conv_dim + ch;
      const float x = Act<T>::load(A.qkv, idx);
      win[K - 1] = x;
      float acc = 0.f;
      for (int j = 0; j < K; ++j) acc = fmaf(w[j], win[j], acc);
      Act<T>::store(A.conv_out, idx, Act<T>::round(silu_f(Act<T>::round(acc))));
      for (int j = 0; j < K - 1; ++j) win[j] = win[j + 1];
    }
    // the last K-1 inputs of the chunk (or of history, when S < K-1) go to their slots
    for (int t = max(0, A.seq - (K - 1)); t < A.seq; ++t) {
      const long idx = ((long)b * A.seq + t) * A.conv_dim + ch;
      Act<T>::store(ring, (pos0 + t) % K, Act<T>::load(A.qkv, idx));
    }
    return;
  }
  const long gg = gid - n_conv;
  if (gg < (long)A.batch * A.seq * A.hv) {
    const int h = gg % A.hv;
    const float beta = Act<T>::round(sigmoid_f(Act<T>::load(A.b, gg)));
    const float ga = Act<T>::load(A.a, gg) + A.dt_bias[h];
    A.beta_out[gg] = beta;
    A.g_out[gg] = A.a_neg[h] * softplus_f(ga);
  }
}

// out = round_T(w * (o * rsqrt(mean(o^2) + eps)) * sigmoid(z)) per 128-row
template <typename T>
__global__ __launch_bounds__(256) void dn_gated_norm_kernel(const T* o, const T* z, const float* w, T* out, long rows,
                                                            float eps) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float o0 = Act<T>::load(o, row * DN_D + lane), o1 = Act<T>::load(o, row * DN_D + 64 + lane);
  const float ss = wave_sum(o0 * o0 + o1 * o1);
  const float rn = rsqrt_rn(ss / (float)DN_D + eps);
  const float z0 = sigmoid_f(Act<T>::load(z, row * DN_D + lane));
  const float z1 = sigmoid_f(Act<T>::load(z, row * DN_D + 64 + lane));
  Act<T>::store(out, row * DN_D + lane, (w[lane] * (o0 * rn)) * z0);
  Act<T>::store(out, row * DN_D + 64 + lane, (w[64 + lane] * (o1 * rn)) * z1);
}

struct PrefillWs {
  size_t conv, g, beta, core, total;
};

PrefillWs prefill_layout(const qm_dn_geom* g, int seq) {
  const size_t act = g->act_dtype == QM_ACT_F32 ? 4 : 2;
  const size_t conv_dim = (size_t)(2 * g->n_k_heads + g->n_v_heads) * g->head_dim;
  PrefillWs w;
  w.conv = 0;
  w.g = w.conv + qm_align256((size_t)g->batch * seq * conv_dim * act);
  w.beta = w.g + qm_align256((size_t)g->batch * seq * g->n_v_heads * 4);
  w.core = w.beta + qm_align256((size_t)g->batch * seq * g->n_v_heads * 4);
  w.total = w.core + qm_align256((size_t)g->batch * seq * g->n_v_heads * g->head_dim * act);
  return w;
}

template <typename T>
int launch_prefill(const qm_dn_geom* g, int seq, const void* qkv, const void* z, const void* a, const void* b,
                   const float* a_neg, const float* dt_bias, const void* conv_w, const float* norm_w,
                   const int* positions, void* conv_ring, float* state, void* out, void* ws, hipStream_t stream) {
  const PrefillWs L = prefill_layout(g, seq);
  char* base = static_cast<char*>(ws);
  T* conv_out = reinterpret_cast<T*>(base + L.conv);
  float* g_out = reinterpret_cast<float*>(base + L.g);
  float* beta_out = reinterpret_cast<float*>(base + L.beta);
  T* core = reinterpret_cast<T*>(base + L.core);
  const int conv_dim = (2 * g->n_k_heads + g->n_v_heads) * DN_D;

  ConvChunkArgs<T> C;
  C.qkv = static_cast<const T*>(qkv); C.a = static_cast<const T*>(a); C.b = static_cast<const T*>(b);
  C.a_neg = a_neg; C.dt_bias = dt_bias; C.conv_w = static_cast<const T*>(conv_w); C.positions = positions;
  C.ring = static_cast<T*>(conv_ring); C.conv_out = conv_out; C.g_out = g_out; C.beta_out = beta_out;
  C.batch = g->batch; C.seq = seq; C.conv_dim = conv_dim; C.K = g->conv_kernel; C.hv = g->n_v_heads;
  const long work = (long)g->batch * conv_dim + (long)g->batch * seq * g->n_v_heads;
  hipLaunchKernelGGL(dn_conv_chunk_kernel<T>, dim3((work + 255) / 256), dim3(256), 0, stream, C);
  QM_CHECK_LAUNCH();

  const int key_dim = g->n_k_heads * DN_D;
  int rc = qm_dn_rule_chunk(g->act_dtype, g->batch, seq, g->n_v_heads, g->n_k_heads, conv_dim, conv_dim, conv_out,
                            conv_out + key_dim, conv_out + 2 * key_dim, g_out, beta_out, state, core, stream);
  if (rc) return rc;

  const long rows = (long)g->batch * seq * g->n_v_heads;
  hipLaunchKernelGGL(dn_gated_norm_kernel<T>, dim3((rows + 3) / 4), dim3(256), 0, stream, core,
                     static_cast<const T*>(z), norm_w, static_cast<T*>(out), rows, g->eps);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

}  // namespace

extern "C" size_t qm_dn_prefill_workspace(const qm_dn_geom* g, int seq) {
  if (!g || seq <= 0) return 0;
  return prefill_layout(g, seq).total;
}

extern "C" int qm_dn_prefill(const qm_dn_geom* g, int seq, const void* qkv, const void* z, const void* a,
                             const void* b, const float* a_neg, const float* dt_bias, const void* conv_w,
                             const float* norm_w, const int* positions, void* conv_ring, float* state, void* out,
                             void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!g) return qm_fail(QM_ERR_ARG, "qm_dn_prefill: null geometry");
  if (g->head_dim != DN_D) return qm_fail(QM_ERR_UNSUPPORTED, "qm_dn_prefill: head_dim must be 128");
  if (g->batch <= 0 || seq <= 0 || g->n_v_heads <= 0 || g->n_k_heads <= 0 || g->n_v_heads % g->n_k_heads)
    return qm_fail(QM_ERR_ARG, "qm_dn_prefill: bad sizes");
  if (g->conv_kernel < 2 || g->conv_kernel > 8) return qm_fail(QM_ERR_ARG, "qm_dn_prefill: conv_kernel must be 2..8");
  if (!qkv || !z || !a || !b || !a_neg || !dt_bias || !conv_w || !norm_w || !positions || !conv_ring || !state || !out)
    return qm_fail(QM_ERR_ARG, "qm_dn_prefill: null tensor pointer");
  if (!workspace || workspace_bytes < qm_dn_prefill_workspace(g, seq))
    return qm_fail(QM_ERR_WORKSPACE, "qm_dn_prefill: workspace too small");
  if (g->act_dtype == QM_ACT_F32)
    return launch_prefill<float>(g, seq, qkv, z, a, b, a_neg, dt_bias, conv_w, norm_w, positions, conv_ring, state,
                                 out, workspace, stream);
  if (g->act_dtype == QM_ACT_BF16)
    return launch_prefill<bf16_t>(g, seq, qkv, z, a, b, a_neg, dt_bias, conv_w, norm_w, positions, conv_ring, state,
                                  out, workspace, stream);
  return qm_fail(QM_ERR_DTYPE, "qm_dn_prefill: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
}
