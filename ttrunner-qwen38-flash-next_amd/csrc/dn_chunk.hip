// Delta rule over a prefill chunk: dispatch between the chunked and token-loop
// kernels.
#include "common.h"
#include "qwen4mix_internal.h"

int qm_dn_rule_chunk(int act_dtype, int batch, int seq, int heads, int hk, long q_stride, long v_stride,
                     const void* q, const void* k, const void* v, const float* g, const float* beta, float* state,
                     void* out, hipStream_t stream) {
  return qm_dn_recurrent_strided(act_dtype, batch, seq, heads, hk, q_stride, v_stride, q, k, v, g, beta, state, out,
                                 stream);
}

extern "C" int qm_dn_chunked(int act_dtype, int batch, int seq, int heads, int head_dim, const void* q, const void* k,
                             const void* v, const float* g, const float* beta, float* state, void* out,
                             hipStream_t stream) {
  if (head_dim != 128) return qm_fail(QM_ERR_UNSUPPORTED, "qm_dn_chunked: head_dim must be 128");
  if (batch <= 0 || seq < 0 || heads <= 0) return qm_fail(QM_ERR_ARG, "qm_dn_chunked: bad sizes");
  if (!q || !k || !v || !g || !beta || !state || !out) return qm_fail(QM_ERR_ARG, "qm_dn_chunked: null pointer");
  if (seq == 0) return QM_OK;
  if (act_dtype != QM_ACT_F32 && act_dtype != QM_ACT_BF16)
    return qm_fail(QM_ERR_DTYPE, "qm_dn_chunked: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
  return qm_dn_rule_chunk(act_dtype, batch, seq, heads, heads, (long)heads * head_dim, (long)heads * head_dim, q, k, v,
                          g, beta, state, out, stream);
}
