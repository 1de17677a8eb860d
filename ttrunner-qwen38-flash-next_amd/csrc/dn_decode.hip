// Gated DeltaNet decode on gfx950: one token per sequence, one launch.
//
// Computes, for every sequence b and value head h (reference/model.py:189-243,
// reference/layers.py:141-147, 155-192, 46-61):
//   conv   : y = silu(sum_t w[c,t] * hist[c,t])  over [ring | x], tap 0 oldest
//   gates  : beta = sigmoid(b), g = A * softplus(a + dt_bias)
//   norms  : q^ = l2norm(q) / sqrt(d), k^ = l2norm(k)   (eps 1e-6)
//   update : S <- S e^g ; pred = S^T k^ ; delta = (v - pred) beta ;
//            S <- S + k^ delta^T ; o = S^T q^  (= q^T S_dec + (q^.k^) delta)
//   norm   : out = rms_norm(o) * w * sigmoid(z)
// with v-head h reading q/k head h % Hk (the tiled layout of the checkpoint).
//
// Work split: 4 workgroups of 256 threads per (sequence, value head), each
// holding 32 of the head's 128 state columns (16 KB of float32, whole 128-byte
// lines of every row): the delta rule is independent per column, so a
// workgroup updates its columns alone and a compute unit moves 32 KB instead
// of the head's 128 KB. Each workgroup recomputes the conv of the head's q/k
// channels (L2-resident) and convolves its own 32 v channels. The gated RMS
// norm needs the head's sum of squares of o: each workgroup publishes its 32
// columns' share in one 64-bit atomic exchange that carries the launch's
// generation number, writes its state columns back, then polls the head's 4
// shares (one cache line) and normalises its columns. All loads are issued at
// the start, the conv's first.
//
// The conv window is a ring of K slots per channel: the input of the token at
// position p lives in slot p % K, so the K-1 history slots read by this step are
// never the slot it writes, and no workgroup can observe another's write.

#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int DN_D = 128;      // head dim (k and v)
constexpr int DN_TILE = 16;    // state columns per workgroup
constexpr int DN_NT = 256;     // threads per workgroup
constexpr int DN_DCOLS = 32;   // state columns per decode workgroup (whole 128-byte lines)
constexpr int DN_SLICES = DN_D / DN_DCOLS;  // decode workgroups per head
// per (sequence, head) a 128-byte line of the decode workspace: the generation
// word, a give-up counter, then the slices' (generation, sum of squares) words
constexpr int DN_SYNC_WORDS = 32;
constexpr int DN_SHARE0 = 4;   // first share, in 64-bit words

template <typename T>
struct DnDecodeArgs {
  const T* qkv; const T* z; const T* a; const T* b;
  const float* a_neg; const float* dt_bias;
  const T* conv_w; const float* norm_w;
  const int* positions;
  T* ring; float* state; T* out;
  unsigned* sync;                  // DN_SYNC_WORDS per (sequence, head)
  int batch, hv, hk, conv_dim, K;
  float eps;
};

// K = 4: the ring row and the weight row of a channel are one 8-byte (bf16) or
// 16-byte (fp32) load each, issued together with the input
template <typename T> struct Vec4;
template <> struct Vec4<float> { typedef float4 type; };
template <> struct Vec4<bf16_t> { typedef uint2 type; };
__device__ __forceinline__ float vget(const float4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
__device__ __forceinline__ float vget(const uint2& v, int i) {
  const unsigned w = i < 2 ? v.x : v.y;
  return bf16_to_f32(static_cast<uint16_t>((i & 1) ? (w >> 16) : (w & 0xffffu)));
}

// A channel's conv inputs (K = 4): its ring row and weight row (one 8-byte or
// 16-byte load each) and the token's input, loaded before any is used.
template <typename T>
struct ConvIn {
  typename Vec4<T>::type r, w;
  float x;
};
template <typename T>
__device__ __forceinline__ ConvIn<T> conv_load4(const DnDecodeArgs<T>& A, int b, int ch) {
  typedef typename Vec4<T>::type V;
  ConvIn<T> c;
  c.r = *reinterpret_cast<const V*>(A.ring + ((long)b * A.conv_dim + ch) * 4);
  c.w = *reinterpret_cast<const V*>(A.conv_w + (long)ch * 4);
  c.x = Act<T>::load(A.qkv, (long)b * A.conv_dim + ch);
  return c;
}
template <typename T>
__device__ __forceinline__ float conv_finish4(const DnDecodeArgs<T>& A, const ConvIn<T>& c, int b, int ch, int pos,
                                              bool write_ring) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 3; ++j) acc = fmaf(vget(c.w, j), vget(c.r, (pos + 1 + j) & 3), acc);
  acc = fmaf(vget(c.w, 3), c.x, acc);
  if (write_ring) Act<T>::store(A.ring + ((long)b * A.conv_dim + ch) * 4, pos & 3, c.x);
  return Act<T>::round(silu_f(Act<T>::round(acc)));
}

template <typename T>
__device__ __forceinline__ float conv_channel(const DnDecodeArgs<T>& A, int b, int ch, int pos, bool write_ring) {
  const int K = A.K;
  const T* w = A.conv_w + (long)ch * K;
  T* ring = A.ring + ((long)b * A.conv_dim + ch) * K;
  const float x = Act<T>::load(A.qkv, (long)b * A.conv_dim + ch);
  float acc = 0.f;
  for (int j = 0; j < K - 1; ++j) {
    int slot = (pos - (K - 1) + j) % K;
    if (slot < 0) slot += K;
    acc = fmaf(Act<T>::load(w, j), Act<T>::load(ring, slot), acc);
  }
  acc = fmaf(Act<T>::load(w, K - 1), x, acc);
  if (write_ring) Act<T>::store(ring, pos % K, x);
  const float y = Act<T>::round(acc);
  return Act<T>::round(silu_f(y));
}

// grid: batch * hv * DN_SLICES workgroups of DN_NT threads; workgroup (b, h, s)
// owns columns 32s..32s+31. Thread t holds rows t/8 + 32k (k = 0..3) of
// columns 32s + 4(t%8)..+3: a wave reads 8 whole rows' lines per load.
template <typename T>
__global__ __launch_bounds__(DN_NT) void dn_decode_kernel(DnDecodeArgs<T> A) {
  const int s = blockIdx.x % DN_SLICES;
  const int h = (blockIdx.x / DN_SLICES) % A.hv;
  const int b = blockIdx.x / (DN_SLICES * A.hv);
  const int hk = h % A.hk;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c8 = tid & 7, r = tid >> 3;
  const int col0 = s * DN_DCOLS;
  constexpr int NW = DN_NT / 64;

  QM_PHASE_DECL
  QM_PHASE(0);
  __shared__ float s_q[DN_D], s_k[DN_D], s_v[DN_DCOLS];
  __shared__ float s_red[NW][2 * DN_DCOLS];
  __shared__ __attribute__((aligned(16))) float s_delta[DN_DCOLS];
  __shared__ float s_w3[2][3];
  __shared__ float s_scal[2];

  // ---- loads, all issued before any is used: the conv inputs of q/k channel
  // t (and of v column t < 32), the position, the gates, z, the norm weight,
  // the state columns and last the generation word (needed last)
  unsigned* line = A.sync + (long)(b * A.hv + h) * DN_SYNC_WORDS;
  unsigned long long* shares = reinterpret_cast<unsigned long long*>(line) + DN_SHARE0;
  const int key_dim = A.hk * DN_D;
  const int ch_qk = tid < DN_D ? hk * DN_D + tid : key_dim + hk * DN_D + (tid - DN_D);
  const int jt = tid & (DN_DCOLS - 1);
  const int ch_v = 2 * key_dim + h * DN_D + col0 + jt;
  const bool k4 = A.K == 4;
  ConvIn<T> cin_qk, cin_v;
  if (k4) {
    cin_qk = conv_load4(A, b, ch_qk);
    cin_v = conv_load4(A, b, ch_v);
  }
  const int pos = A.positions[b];
  const float gate_b = Act<T>::load(A.b, (long)b * A.hv + h), gate_a = Act<T>::load(A.a, (long)b * A.hv + h);
  const float a_neg = A.a_neg[h], dtb = A.dt_bias[h];
  const float zv = Act<T>::load(A.z, (long)b * A.hv * DN_D + h * DN_D + col0 + jt);
  const float nw = A.norm_w[col0 + jt];
  float4* S = reinterpret_cast<float4*>(A.state + ((long)(b * A.hv + h) * DN_D) * DN_D) + col0 / 4 + c8;
  float4 st4[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) st4[k] = S[(r + 32 * k) * (DN_D / 4)];
  const unsigned gen = ld_flag(line);

  // ---- conv: q/k channel t (one writer of each q/k channel's ring slot: the
  // first slice of the head with h == hk), v column t < 32; then the gates
  const bool qk_writer = h == hk && s == 0;
  const float y_qk = k4 ? conv_finish4(A, cin_qk, b, ch_qk, pos, qk_writer) : conv_channel(A, b, ch_qk, pos, qk_writer);
  (tid < DN_D ? s_q[tid] : s_k[tid - DN_D]) = y_qk;
  if (tid < DN_DCOLS) s_v[tid] = k4 ? conv_finish4(A, cin_v, b, ch_v, pos, true) : conv_channel(A, b, ch_v, pos, true);
  if (tid == 0) {
    s_scal[0] = Act<T>::round(sigmoid_f(gate_b));
    s_scal[1] = expf(a_neg * softplus_f(gate_a + dtb));
  }
  __syncthreads();

  QM_PHASE(1);
  // ---- l2 norms of q and k and their dot product: waves 0-1 hold the 128 channels
  if (tid < DN_D) {
    const float qv = s_q[tid], kv = s_k[tid];
    const float a0 = wave_sum(qv * qv), a1 = wave_sum(kv * kv), a2 = wave_sum(qv * kv);
    if (lane == 0) { s_w3[wid][0] = a0; s_w3[wid][1] = a1; s_w3[wid][2] = a2; }
  }
  __syncthreads();
  const float sq = s_w3[0][0] + s_w3[1][0], sk = s_w3[0][1] + s_w3[1][1], sqk = s_w3[0][2] + s_w3[1][2];
  const float rq = rsqrt_rn(sq + 1e-6f), rk = rsqrt_rn(sk + 1e-6f);
  const float sqrt_d = 11.313708498984761f;
  const float qk = div_rn(sqk * rq * rk, sqrt_d);       // q^ . k^

  QM_PHASE(2);
  // ---- decay, then per column pred = S^T k^ and qd = S^T q^ over the rows
  const float decay = s_scal[1];
  float st[4][4], kr[4], pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int row = r + 32 * k;
    kr[k] = mul_rn(s_k[row], rk);
    const float qr = div_rn(mul_rn(s_q[row], rq), sqrt_d);
    st[k][0] = st4[k].x * decay; st[k][1] = st4[k].y * decay;
    st[k][2] = st4[k].z * decay; st[k][3] = st4[k].w * decay;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      pk[c] = fmaf(st[k][c], kr[k], pk[c]);
      pq[c] = fmaf(st[k][c], qr, pq[c]);
    }
  }
  // the 8 lanes of one c8 in a wave: lane ^ 8 within a 16-lane row (rotation
  // by 8), then across the rows
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    pk[c] += dpp_f<0x128>(pk[c]);
    pk[c] = xor32_sum(xor16_sum(pk[c]));
    pq[c] += dpp_f<0x128>(pq[c]);
    pq[c] = xor32_sum(xor16_sum(pq[c]));
  }
  if (lane < 8) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s_red[wid][4 * lane + c] = pk[c];
      s_red[wid][DN_DCOLS + 4 * lane + c] = pq[c];
    }
  }
  __syncthreads();

  QM_PHASE(3);
  // ---- delta and o of the 32 columns (wave 0, lanes 0-31); their share of the
  // head's sum of squares leaves at once
  float o = 0.f;
  if (tid < DN_DCOLS) {
    float pred = 0.f, qd = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) { pred += s_red[w][tid]; qd += s_red[w][DN_DCOLS + tid]; }
    const float delta = (s_v[tid] - pred) * s_scal[0];
    s_delta[tid] = delta;
    o = Act<T>::round(fmaf(qk, delta, qd));
  }
  if (wid == 0) {
    const float ss = xor16_sum(row16_sum(tid < DN_DCOLS ? o * o : 0.f));
    if (lane == 0) {
      const unsigned long long word = ((unsigned long long)(gen + 1) << 32) | __float_as_uint(ss);
      raise_word(shares + s, word);
    }
  }
  __syncthreads();

  QM_PHASE(4);
  // ---- rank-1 update and write-back of the columns, written through to the
  // point of coherence: no dirty state lines are left in L2 for the end of
  // the kernel to write back (0.35 µs less per launch)
  {
    const float4 dl = *reinterpret_cast<const float4*>(s_delta + 4 * c8);
    const __amdgpu_buffer_rsrc_t rs = dev_rsrc(A.state + ((long)(b * A.hv + h) * DN_D) * DN_D, DN_D * DN_D * 4);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      st_dev4(rs, ((r + 32 * k) * DN_D + col0 + 4 * c8) * 4,
              make_float4(fmaf(kr[k], dl.x, st[k][0]), fmaf(kr[k], dl.y, st[k][1]), fmaf(kr[k], dl.z, st[k][2]),
                          fmaf(kr[k], dl.w, st[k][3])));
  }

  QM_PHASE(5);
  // ---- the head's sum of squares from its shares (one line, polled by wave
  // 0), then the gated RMS norm of the 32 columns
  if (wid == 0) {
    float ss_all = 0.f;
    bool done = false;
    for (int it = 0; it < FLAG_SPIN_MAX && !done; ++it) {
      const unsigned long long w =
          __hip_atomic_load(shares + (lane & (DN_SLICES - 1)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool ok = (int)((unsigned)(w >> 32) - (gen + 1)) >= 0;
      if (__builtin_amdgcn_ballot_w64(!ok) == 0ull) {
        const float v = __uint_as_float((unsigned)w);
#pragma unroll
        for (int k = 0; k < DN_SLICES; ++k) ss_all += readlane_f(v, k);
        done = true;
      } else {
        __builtin_amdgcn_s_sleep(1);
      }
    }
    // a wait that gave up counts itself (qm_dn_decode_check) and leaves NaN,
    // never an output normalised by a partial sum
    QM_PHASE(6);
    if (!done && lane == 0) __hip_atomic_fetch_add(line + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (s == 0 && lane == 0) st_flag(line, gen + 1);
    if (tid < DN_DCOLS) {
      const float rn = rsqrt_rn(ss_all / (float)DN_D + A.eps);
      const float y = (nw * (o * rn)) * sigmoid_f(zv);
      Act<T>::store(A.out, (long)b * A.hv * DN_D + h * DN_D + col0 + tid, done ? y : __builtin_nanf(""));
    }
  }
  QM_PHASE(7);
  QM_PHASE_FLUSH();
}

// ---------------------------------------------------------------------------
// Multi-token recurrence on already split and expanded q, k, v (the free
// function recurrent_gated_delta_rule, reference/layers.py:155-192). Same
// column split; the state tile stays in registers across the T tokens.
// ---------------------------------------------------------------------------
template <typename T>
struct DnRecurArgs {
  const T* q; const T* k; const T* v;       // token rows of q_stride / v_stride elements
  const float* g; const float* beta;        // [B, T, H]
  float* state;                             // [B, H, D, D]
  T* out;                                   // [B, T, H, D]
  int batch, seq, heads, hk;                // head h reads q/k head h % hk
  long q_stride, v_stride;
};

template <typename T>
__global__ __launch_bounds__(DN_NT) void dn_recurrent_kernel(DnRecurArgs<T> A) {
  constexpr int NTILE = DN_D / DN_TILE;
  const int nwg = A.batch * A.heads * NTILE;
  const int wg = xcd_remap(blockIdx.x, nwg);
  const int tile = wg % NTILE;
  const int h = (wg / NTILE) % A.heads;
  const int b = wg / (NTILE * A.heads);
  const int col0 = tile * DN_TILE;
  const int tid = threadIdx.x;
  const int c4 = tid & 3, r = tid >> 2;
  const int lane = tid & 63, wid = tid >> 6;

  __shared__ float s_q[DN_D], s_k[DN_D], s_v[DN_TILE];
  __shared__ float s_red[4][2 * DN_TILE];
  __shared__ float s_delta[DN_TILE];
  __shared__ float s_scal[4];
  __shared__ float s_wred[DN_NT / 64];

  float4* S = reinterpret_cast<float4*>(A.state + ((long)(b * A.heads + h) * DN_D) * DN_D);
  const int rowf4 = DN_D / 4;
  float4 s0 = S[r * rowf4 + col0 / 4 + c4];
  float4 s1 = S[(r + 64) * rowf4 + col0 / 4 + c4];
  float st0[4] = {s0.x, s0.y, s0.z, s0.w};
  float st1[4] = {s1.x, s1.y, s1.z, s1.w};
  const float inv_sqrt_d = 11.313708498984761f;

  for (int t = 0; t < A.seq; ++t) {
    const long tok = (long)b * A.seq + t;
    const long row = tok * A.heads + h;
    const int i = tid & (DN_D - 1);
    const long qoff = tok * A.q_stride + (long)(h % A.hk) * DN_D + i;
    const float qv = Act<T>::load(A.q, qoff);
    const float kv = Act<T>::load(A.k, qoff);
    if (tid < DN_TILE) s_v[tid] = Act<T>::load(A.v, tok * A.v_stride + (long)h * DN_D + col0 + tid);
    float sq = tid < DN_D ? qv * qv : 0.f;
    float sk = tid < DN_D ? kv * kv : 0.f;
    float sqk = tid < DN_D ? qv * kv : 0.f;
    sq = block_sum<DN_NT>(sq, s_wred);
    sk = block_sum<DN_NT>(sk, s_wred);
    sqk = block_sum<DN_NT>(sqk, s_wred);
    const float rq = rsqrt_rn(sq + 1e-6f), rk = rsqrt_rn(sk + 1e-6f);
    if (tid < DN_D) {
      s_q[tid] = div_rn(mul_rn(qv, rq), inv_sqrt_d);
      s_k[tid] = mul_rn(kv, rk);
    }
    if (tid == 0) {
      s_scal[0] = A.beta[row];
      s_scal[1] = expf(A.g[row]);
      s_scal[2] = div_rn(sqk * rq * rk, inv_sqrt_d);
    }
    __syncthreads();
    const float decay = s_scal[1];
    const float kr0 = s_k[r], kr1 = s_k[r + 64], qr0 = s_q[r], qr1 = s_q[r + 64];
    float pk[4], pq[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      st0[c] *= decay;
      st1[c] *= decay;
      pk[c] = fmaf(st0[c], kr0, st1[c] * kr1);
      pq[c] = fmaf(st0[c], qr0, st1[c] * qr1);
    }
#pragma unroll
    for (int off = 4; off < 64; off <<= 1) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        pk[c] += __shfl_xor(pk[c], off, 64);
        pq[c] += __shfl_xor(pq[c], off, 64);
      }
    }
    if (lane < 4) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s_red[wid][lane * 4 + c] = pk[c];
        s_red[wid][DN_TILE + lane * 4 + c] = pq[c];
      }
    }
    __syncthreads();
    if (tid < DN_TILE) {
      const float pred = s_red[0][tid] + s_red[1][tid] + s_red[2][tid] + s_red[3][tid];
      const float qd = s_red[0][DN_TILE + tid] + s_red[1][DN_TILE + tid] + s_red[2][DN_TILE + tid] +
                       s_red[3][DN_TILE + tid];
      const float delta = (s_v[tid] - pred) * s_scal[0];
      s_delta[tid] = delta;
      Act<T>::store(A.out, row * DN_D + col0 + tid, fmaf(s_scal[2], delta, qd));
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float dl = s_delta[c4 * 4 + c];
      st0[c] = fmaf(kr0, dl, st0[c]);
      st1[c] = fmaf(kr1, dl, st1[c]);
    }
  }
  S[r * rowf4 + col0 / 4 + c4] = make_float4(st0[0], st0[1], st0[2], st0[3]);
  S[(r + 64) * rowf4 + col0 / 4 + c4] = make_float4(st1[0], st1[1], st1[2], st1[3]);
}

template <typename T>
int launch_dn_decode(const qm_dn_geom* g, const void* qkv, const void* z, const void* a, const void* b,
                     const float* a_neg, const float* dt_bias, const void* conv_w, const float* norm_w,
                     const int* positions, void* conv_ring, float* state, void* out, void* ws,
                     hipStream_t stream) {
  DnDecodeArgs<T> A;
  A.qkv = static_cast<const T*>(qkv); A.z = static_cast<const T*>(z);
  A.a = static_cast<const T*>(a); A.b = static_cast<const T*>(b);
  A.a_neg = a_neg; A.dt_bias = dt_bias;
  A.conv_w = static_cast<const T*>(conv_w); A.norm_w = norm_w;
  A.positions = positions;
  A.ring = static_cast<T*>(conv_ring); A.state = state; A.out = static_cast<T*>(out);
  A.batch = g->batch; A.hv = g->n_v_heads; A.hk = g->n_k_heads;
  A.conv_dim = 2 * g->n_k_heads * DN_D + g->n_v_heads * DN_D;
  A.K = g->conv_kernel; A.eps = g->eps;
  A.sync = static_cast<unsigned*>(ws);
  const int nwg = g->batch * g->n_v_heads * DN_SLICES;
  hipLaunchKernelGGL(dn_decode_kernel<T>, dim3(nwg), dim3(DN_NT), 0, stream, A);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

template <typename T>
int launch_dn_recurrent(int batch, int seq, int heads, int hk, long q_stride, long v_stride, const void* q,
                        const void* k, const void* v, const float* g, const float* beta, float* state, void* out,
                        hipStream_t stream) {
  DnRecurArgs<T> A;
  A.q = static_cast<const T*>(q); A.k = static_cast<const T*>(k); A.v = static_cast<const T*>(v);
  A.g = g; A.beta = beta; A.state = state; A.out = static_cast<T*>(out);
  A.batch = batch; A.seq = seq; A.heads = heads; A.hk = hk; A.q_stride = q_stride; A.v_stride = v_stride;
  const int nwg = batch * heads * (DN_D / DN_TILE);
  hipLaunchKernelGGL(dn_recurrent_kernel<T>, dim3(nwg), dim3(DN_NT), 0, stream, A);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

}  // namespace

QM_PHASE_ENTRY(dn)

extern "C" size_t qm_dn_decode_workspace(int batch, int n_v_heads, int head_dim) {
  // one 128-byte line per (sequence, head): generation word and the shares of
  // the gated norm's sum of squares
  if (batch <= 0 || n_v_heads <= 0 || head_dim <= 0) return 0;
  return qm_align256((size_t)batch * n_v_heads * DN_SYNC_WORDS * sizeof(unsigned));
}

extern "C" int qm_dn_decode_check(int batch, int n_v_heads, int head_dim, void* workspace, size_t workspace_bytes,
                                  int reset, unsigned* giveups, hipStream_t stream) {
  if (!workspace || !giveups) return qm_fail(QM_ERR_ARG, "qm_dn_decode_check: null pointer");
  const size_t need = qm_dn_decode_workspace(batch, n_v_heads, head_dim);
  if (need == 0 || workspace_bytes < need) return qm_fail(QM_ERR_WORKSPACE, "qm_dn_decode_check: workspace too small");
  const long n_lines = (long)batch * n_v_heads;
  unsigned* host = new unsigned[n_lines * DN_SYNC_WORDS];
  hipError_t e = hipMemcpyAsync(host, workspace, n_lines * DN_SYNC_WORDS * sizeof(unsigned), hipMemcpyDeviceToHost,
                                stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    delete[] host;
    return qm_fail(QM_ERR_LAUNCH, hipGetErrorString(e));
  }
  *giveups = 0;
  for (long i = 0; i < n_lines; ++i) *giveups += host[i * DN_SYNC_WORDS + 1];
  delete[] host;
  return reset ? qm_zero_words(workspace, n_lines * DN_SYNC_WORDS, stream) : QM_OK;
}

extern "C" int qm_dn_decode(const qm_dn_geom* g, const void* qkv, const void* z, const void* a, const void* b,
                            const float* a_neg, const float* dt_bias, const void* conv_w, const float* norm_w,
                            const int* positions, void* conv_ring, float* state, void* out, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
  if (!g) return qm_fail(QM_ERR_ARG, "qm_dn_decode: null geometry");
  if (g->head_dim != DN_D) return qm_fail(QM_ERR_UNSUPPORTED, "qm_dn_decode: head_dim must be 128");
  if (g->batch <= 0 || g->n_v_heads <= 0 || g->n_k_heads <= 0 || g->n_v_heads % g->n_k_heads)
    return qm_fail(QM_ERR_ARG, "qm_dn_decode: need batch > 0 and n_v_heads a multiple of n_k_heads");
  if (g->conv_kernel < 2 || g->conv_kernel > 8) return qm_fail(QM_ERR_ARG, "qm_dn_decode: conv_kernel must be 2..8");
  if (!qkv || !z || !a || !b || !a_neg || !dt_bias || !conv_w || !norm_w || !positions || !conv_ring || !state || !out)
    return qm_fail(QM_ERR_ARG, "qm_dn_decode: null tensor pointer");
  if (!workspace || workspace_bytes < qm_dn_decode_workspace(g->batch, g->n_v_heads, g->head_dim))
    return qm_fail(QM_ERR_WORKSPACE, "qm_dn_decode: workspace too small");
  if (g->act_dtype == QM_ACT_F32)
    return launch_dn_decode<float>(g, qkv, z, a, b, a_neg, dt_bias, conv_w, norm_w, positions, conv_ring, state, out,
                                   workspace, stream);
  if (g->act_dtype == QM_ACT_BF16)
    return launch_dn_decode<bf16_t>(g, qkv, z, a, b, a_neg, dt_bias, conv_w, norm_w, positions, conv_ring, state, out,
                                    workspace, stream);
  return qm_fail(QM_ERR_DTYPE, "qm_dn_decode: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
}

extern "C" int qm_dn_recurrent(int act_dtype, int batch, int seq, int heads, int head_dim, const void* q,
                               const void* k, const void* v, const float* g, const float* beta, float* state,
                               void* out, hipStream_t stream) {
  if (head_dim != DN_D) return qm_fail(QM_ERR_UNSUPPORTED, "qm_dn_recurrent: head_dim must be 128");
  if (batch <= 0 || seq < 0 || heads <= 0) return qm_fail(QM_ERR_ARG, "qm_dn_recurrent: bad sizes");
  if (!q || !k || !v || !g || !beta || !state || !out) return qm_fail(QM_ERR_ARG, "qm_dn_recurrent: null pointer");
  if (seq == 0) return QM_OK;
  return qm_dn_recurrent_strided(act_dtype, batch, seq, heads, heads, (long)heads * head_dim, (long)heads * head_dim,
                                 q, k, v, g, beta, state, out, stream);
}

int qm_dn_recurrent_strided(int act_dtype, int batch, int seq, int heads, int hk, long q_stride, long v_stride,
                            const void* q, const void* k, const void* v, const float* g, const float* beta,
                            float* state, void* out, hipStream_t stream) {
  if (act_dtype == QM_ACT_F32)
    return launch_dn_recurrent<float>(batch, seq, heads, hk, q_stride, v_stride, q, k, v, g, beta, state, out, stream);
  if (act_dtype == QM_ACT_BF16)
    return launch_dn_recurrent<bf16_t>(batch, seq, heads, hk, q_stride, v_stride, q, k, v, g, beta, state, out,
                                       stream);
  return qm_fail(QM_ERR_DTYPE, "qm_dn_recurrent: act_dtype must be QM_ACT_F32 or QM_ACT_BF16");
}
