// Internal declarations shared by the qwen4mix translation units.
#pragma once

#include <stddef.h>

#include "qwen4mix.h"

// Record `msg` as the calling thread's last error and return `code`.
int qm_fail(int code, const char* msg);

inline size_t qm_align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

// The delta-rule token loop over strided q/k/v rows (q/k head h % hk): shared
// by qm_dn_recurrent and the prefill path.
int qm_dn_recurrent_strided(int act_dtype, int batch, int seq, int heads, int hk, long q_stride, long v_stride,
                            const void* q, const void* k, const void* v, const float* g, const float* beta,
                            float* state, void* out, hipStream_t stream);

// The delta rule over a chunk of tokens for the prefill path: the WY/UT chunked
// kernels (64-token chunks) for chunks of 16 tokens or more, the token loop for
// shorter ones. `ws` holds qm_dn_rule_chunk_workspace(batch, seq, heads) bytes.
size_t qm_dn_rule_chunk_workspace(int batch, int seq, int heads);
int qm_dn_rule_chunk(int act_dtype, int batch, int seq, int heads, int hk, long q_stride, long v_stride,
                     const void* q, const void* k, const void* v, const float* g, const float* beta, float* state,
                     void* out, void* ws, size_t ws_bytes, hipStream_t stream);

// Workgroups of `kernel` (launched with block_threads threads and dyn_lds bytes
// of dynamic LDS) that can be resident on the current device at once: the
// occupancy per compute unit times the compute units. Cached per device.
int qm_resident_workgroups(const void* kernel, int block_threads, size_t dyn_lds, int* out);

// Zero n_words 32-bit words at p with a fill kernel on `stream`.
int qm_zero_words(void* p, long n_words, hipStream_t stream);
