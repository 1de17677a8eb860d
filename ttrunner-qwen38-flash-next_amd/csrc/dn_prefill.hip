// Gated DeltaNet over a chunk of S tokens (prefill), gfx950.
//
// The seq > 1 body of Qwen4ExpModel._linear_attention (reference/model.py:
// 198-201, 205-217, 230-243): the causal conv over [history | chunk] with the
// last K-1 inputs carried to the ring, the gates, the delta rule over the chunk,
// and the gated RMS norm. Launches:
//   dn_conv_chunk   a workgroup per (sequence, 16 tokens, 256 channels): each
//                   thread loads its channel's window inputs at once, then
//                   writes 16 outputs; the first token block writes the ring;
//                   the same grid computes beta and g for every (token, head)
//   delta rule      the WY/UT chunked kernels (dn_chunk.hip) for chunks of 16
//                   tokens or more, the token loop for shorter ones
//   dn_gated_norm   one wavefront per (token, head) row of 128
#include <atomic>

#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int DN_D = 128;

template <typename T>
struct ConvChunkArgs {
  const T* qkv; const T* a; const T* b; const float* a_neg; const float* dt_bias; const T* conv_w;
  const int* positions; T* ring; T* conv_out; float* g_out; float* beta_out;
  int batch, seq, conv_dim, hv, n_conv_wg;
};

constexpr int CONV_CH = 256;   // channels per workgroup (one per thread)
constexpr int CONV_TOK = 16;   // tokens per workgroup

// Workgroups [0, n_conv_wg) cover (sequence, 16-token block, 256 channels):
// a thread loads its channel's K-1 + 16 inputs up front (history from the ring
// before the chunk's first token), then writes the 16 outputs. The workgroup of
// the first token block alone reads the ring, and it also writes the last K-1
// inputs back to their slots after those reads, so no other workgroup races on
// the ring. The remaining workgroups compute beta and g per (token, head).
template <typename T, int K>
__global__ __launch_bounds__(CONV_CH) void dn_conv_chunk_kernel(ConvChunkArgs<T> A) {
  const int tid = threadIdx.x;
  if ((int)blockIdx.x < A.n_conv_wg) {
    const int n_cb = (A.conv_dim + CONV_CH - 1) / CONV_CH;
    const int n_tb = (A.seq + CONV_TOK - 1) / CONV_TOK;
    const int cb = blockIdx.x % n_cb, tb = (blockIdx.x / n_cb) % n_tb, b = blockIdx.x / (n_cb * n_tb);
    const int ch = cb * CONV_CH + tid;
    if (ch >= A.conv_dim) return;
    // the position first (a scalar load, waited for only where the ring
    // slots are chosen, after every vector load below is issued)
    const int pos0 = A.positions[b];
    const int t0 = tb * CONV_TOK;
    const int nt = min(CONV_TOK, A.seq - t0);
    T* ring = A.ring + ((long)b * A.conv_dim + ch) * K;
    const T* x = A.qkv + (long)b * A.seq * A.conv_dim + ch;
    // every load is unconditional (clamped index, then a select) and none
    // depends on the position, so all are issued before the first wait: the
    // window, the weights and all K ring slots (the history is chosen from
    // them once the position is in)
    float w[K], slots[K], win[CONV_TOK + K - 1];
#pragma unroll
    for (int i = 0; i < CONV_TOK + K - 1; ++i) {
      const int t = t0 - (K - 1) + i;
      win[i] = Act<T>::load(x, (long)min(max(t, 0), A.seq - 1) * A.conv_dim);
    }
#pragma unroll
    for (int j = 0; j < K; ++j) w[j] = Act<T>::load(A.conv_w, (long)ch * K + j);
    // the first token block alone reads the ring (the others load their own
    // column's first input in its place, so none reads a slot it rewrites),
    // and keeps the chunk's last K-1 inputs for it; unconditional, so that
    // these loads go out with the window's
    const T* rsrc = t0 == 0 ? ring : x;
#pragma unroll
    for (int j = 0; j < K; ++j) slots[j] = Act<T>::load(rsrc, t0 == 0 ? j : 0);
    T last[K - 1];
#pragma unroll
    for (int i = 0; i < K - 1; ++i) last[i] = x[(long)max(A.seq - (K - 1) + i, 0) * A.conv_dim];
    // win[i] = input of token t0 - (K-1) + i; tokens before the chunk come
    // from the ring slots (pos0 - (K-1) + i) mod K (first token block)
    // (a select, not a branch: the slot loads then stay with the window's
    // instead of being moved into the branch that uses them)
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
      int slot = (pos0 - (K - 1) + i) % K;
      if (slot < 0) slot += K;
      float h = slots[0];
#pragma unroll
      for (int u = 1; u < K; ++u) h = slot == u ? slots[u] : h;
      win[i] = t0 == 0 ? h : win[i];
    }
#pragma unroll
    for (int i = 0; i < CONV_TOK; ++i) {
      if (i < nt) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) acc = fmaf(w[j], win[i + j], acc);
        Act<T>::store(A.conv_out, ((long)b * A.seq + t0 + i) * A.conv_dim + ch,
                      Act<T>::round(silu_f(Act<T>::round(acc))));
      }
    }
    if (tb == 0) {
      // the last K-1 inputs of the chunk (or all of them, when S < K-1) go to their slots
#pragma unroll
      for (int i = 0; i < K - 1; ++i) {
        const int t = A.seq - (K - 1) + i;
        if (t >= 0) ring[(pos0 + t) % K] = last[i];
      }
    }
    return;
  }
  // (token, head) pairs: the host keeps batch * seq * hv below 2^31
  const int gg = (static_cast<int>(blockIdx.x) - A.n_conv_wg) * CONV_CH + tid;
  if (gg < A.batch * A.seq * A.hv) {
    const int h = gg % A.hv;
    // all four loads before either value is formed (the activations as
    // loaded: a conversion next to its load would wait for it there)
    const T braw = A.b[gg], araw = A.a[gg];
    const float dtb = A.dt_bias[h], an = A.a_neg[h];
    __builtin_amdgcn_sched_barrier(0);
    A.beta_out[gg] = Act<T>::round(sigmoid_f(Act<T>::load(&braw, 0)));
    A.g_out[gg] = an * softplus_fast(Act<T>::load(&araw, 0) + dtb);
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
  size_t conv, g, beta, core, rule, total;
};

PrefillWs prefill_layout(const qm_dn_geom* g, int seq) {
  const size_t act = g->act_dtype == QM_ACT_F32 ? 4 : 2;
  const size_t conv_dim = (size_t)(2 * g->n_k_heads + g->n_v_heads) * g->head_dim;
  PrefillWs w;
  w.conv = 0;
  w.g = w.conv + qm_align256((size_t)g->batch * seq * conv_dim * act);
  w.beta = w.g + qm_align256((size_t)g->batch * seq * g->n_v_heads * 4);
  w.core = w.beta + qm_align256((size_t)g->batch * seq * g->n_v_heads * 4);
  w.rule = w.core + qm_align256((size_t)g->batch * seq * g->n_v_heads * g->head_dim * act);
  w.total = w.rule + qm_align256(qm_dn_rule_chunk_workspace(g->batch, seq, g->n_v_heads));
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
  C.batch = g->batch; C.seq = seq; C.conv_dim = conv_dim; C.hv = g->n_v_heads;
  C.n_conv_wg = g->batch * ((conv_dim + CONV_CH - 1) / CONV_CH) * ((seq + CONV_TOK - 1) / CONV_TOK);
  const long n_gate = (long)g->batch * seq * g->n_v_heads;
  if (n_gate > 0x7fffffffL - CONV_CH)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_dn_prefill: batch * seq * value heads must stay below 2^31");
  const dim3 grid(C.n_conv_wg + (unsigned)((n_gate + CONV_CH - 1) / CONV_CH));
  switch (g->conv_kernel) {
    case 2: hipLaunchKernelGGL((dn_conv_chunk_kernel<T, 2>), grid, dim3(CONV_CH), 0, stream, C); break;
    case 3: hipLaunchKernelGGL((dn_conv_chunk_kernel<T, 3>), grid, dim3(CONV_CH), 0, stream, C); break;
    case 4: hipLaunchKernelGGL((dn_conv_chunk_kernel<T, 4>), grid, dim3(CONV_CH), 0, stream, C); break;
    case 5: hipLaunchKernelGGL((dn_conv_chunk_kernel<T, 5>), grid, dim3(CONV_CH), 0, stream, C); break;
    case 6: hipLaunchKernelGGL((dn_conv_chunk_kernel<T, 6>), grid, dim3(CONV_CH), 0, stream, C); break;
    case 7: hipLaunchKernelGGL((dn_conv_chunk_kernel<T, 7>), grid, dim3(CONV_CH), 0, stream, C); break;
    default: hipLaunchKernelGGL((dn_conv_chunk_kernel<T, 8>), grid, dim3(CONV_CH), 0, stream, C); break;
  }
  QM_CHECK_LAUNCH();

  const int key_dim = g->n_k_heads * DN_D;
  int rc = qm_dn_rule_chunk(g->act_dtype, g->batch, seq, g->n_v_heads, g->n_k_heads, conv_dim, conv_dim, conv_out,
                            conv_out + key_dim, conv_out + 2 * key_dim, g_out, beta_out, state, core, base + L.rule,
                            L.total - L.rule, stream);
  if (rc) return rc;

  const long rows = (long)g->batch * seq * g->n_v_heads;
  hipLaunchKernelGGL(dn_gated_norm_kernel<T>, dim3((rows + 3) / 4), dim3(256), 0, stream, core,
                     static_cast<const T*>(z), norm_w, static_cast<T*>(out), rows, g->eps);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

}  // namespace

// The allocation-free variant's workspace: one array per device, for the
// whole process. Its address on each device comes from hipGetSymbolAddress
// (the array's name in host code is only a stand-in); calls on one device
// share it, so they must not overlap.
constexpr size_t NOALLOC_SCRATCH_BYTES = 32ull << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int NOALLOC_MAX_DEVICES = 64;
std::atomic<void*> g_scratch_ptr[NOALLOC_MAX_DEVICES];

// the current device's address of `scratch`, looked up once per device
int scratch_on_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    return qm_fail(QM_ERR_LAUNCH, "qm_dn_prefill_noalloc: no current HIP device");
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return qm_fail(QM_ERR_LAUNCH, "qm_dn_prefill_noalloc: hipGetSymbolAddress failed");
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return QM_OK;
}

}  // namespace

extern "C" size_t qm_dn_prefill_noalloc_max_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int qm_dn_prefill_noalloc(const qm_dn_geom* g, int seq, const void* qkv, const void* z, const void* a,
                                     const void* b, const float* a_neg, const float* dt_bias, const void* conv_w,
                                     const float* norm_w, const int* positions, void* conv_ring, float* state,
                                     void* out, hipStream_t stream) {
  if (!g) return qm_fail(QM_ERR_ARG, "qm_dn_prefill_noalloc: null geometry");
  if (g->batch <= 0 || seq <= 0) return qm_fail(QM_ERR_ARG, "qm_dn_prefill_noalloc: bad sizes");
  const size_t need = qm_dn_prefill_workspace(g, seq);
  if (need > NOALLOC_SCRATCH_BYTES)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_dn_prefill_noalloc: this batch * seq needs more than the 32 MiB of "
                                       "built-in scratch (about 256 tokens at 32 heads; use qm_dn_prefill with a "
                                       "workspace)");
  void* ws = nullptr;
  const int rc = scratch_on_device(&ws);
  if (rc) return rc;
  return qm_dn_prefill(g, seq, qkv, z, a, b, a_neg, dt_bias, conv_w, norm_w, positions, conv_ring, state, out, ws,
                       NOALLOC_SCRATCH_BYTES, stream);
}

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
