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
// lines of every row, moved by 16-byte loads and stores): the delta rule is
// independent per column, so a workgroup updates its columns alone. Each
// workgroup recomputes the conv of the head's q/k channels and convolves its
// own 32 v channels. The gated RMS norm needs the head's sum of squares of o:
// each workgroup publishes its columns' share in one 64-bit word that carries
// the launch's generation number, writes its state columns back, then polls
// the head's 4 shares (one cache line) and normalises its columns. All loads
// are issued at the start, before any of them is waited for, and stores wait
// for the end (loads and stores share one in-order counter).
//
// Measured (MI355X, batch 1, 32 heads): about 4.2 us per launch back to back
// from a HIP graph, 4.5 us with the state coming from HBM (caches flushed
// before the launch). A workgroup's own span is about 3.6 us of that; the rest
// is the launch's fixed cost. A single 1024-thread workgroup per head needs no
// hand-off but moves 64 KB through one compute unit, and measured 0.5 us
// slower.
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
constexpr int DN_DEC_NT = 256;   // threads per decode workgroup: four float4 of the slice each
constexpr int DN_DCOLS = 32;     // state columns per decode workgroup (whole 128-byte lines)
constexpr int DN_SLICES = DN_D / DN_DCOLS;  // decode workgroups per head
// per (sequence, head) a 128-byte line of the decode workspace: the generation
// word, a give-up counter, then the slices' (generation, sum of squares) words
constexpr int DN_SYNC_WORDS = 32;
constexpr int DN_SHARE0 = 2;     // first share, in 64-bit words


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
// 16-byte load each) and the token's input, kept as loaded (no conversion, so
// nothing waits for them before the kernel's other loads are issued). The
// caller stores the input into the ring slot pos % 4.
template <typename T>
struct ConvIn {
  typename Vec4<T>::type r, w;
  T x;
};
template <typename T>
__device__ __forceinline__ ConvIn<T> conv_load4(const T* ring, const T* conv_w, const T* qkv, int conv_dim, int b,
                                                int ch) {
  typedef typename Vec4<T>::type V;
  ConvIn<T> c;
  c.r = *reinterpret_cast<const V*>(ring + ((long)b * conv_dim + ch) * 4);
  c.w = *reinterpret_cast<const V*>(conv_w + (long)ch * 4);
  c.x = qkv[(long)b * conv_dim + ch];
  return c;
}
template <typename T>
__device__ __forceinline__ float conv_finish4(const ConvIn<T>& c, int pos) {
  const float x = Act<T>::load(&c.x, 0);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 3; ++j) acc = fmaf(vget(c.w, j), vget(c.r, (pos + 1 + j) & 3), acc);
  acc = fmaf(vget(c.w, 3), x, acc);
  return Act<T>::round(silu_f(Act<T>::round(acc)));
}

// Hides a value's origin from the optimiser, so that work on it is not moved
// up to where it was loaded.
__device__ __forceinline__ void opaque(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void opaque(unsigned& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void opaque(bf16_t& v) {
  unsigned u = v.bits;
  asm volatile("" : "+v"(u));
  v.bits = static_cast<uint16_t>(u);
}

// v + the value of lane l ^ 16, in every lane: v_permlane16_swap exchanges the
// odd 16-lane rows of one copy with the even rows of another.
__device__ __forceinline__ float rows_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// the value of lane l ^ 32
__device__ __forceinline__ float halves_swap(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// v + the value of lane l ^ 32, in every lane, without LDS: v_permlane32_swap
// exchanges the upper half of one copy with the lower half of another.
__device__ __forceinline__ float halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <typename T>
__device__ __forceinline__ float conv_channel(T* ring_all, const T* conv_w, const T* qkv, int conv_dim, int K, int b,
                                              int ch, int pos, bool write_ring) {
  const T* w = conv_w + (long)ch * K;
  T* ring = ring_all + ((long)b * conv_dim + ch) * K;
  const float x = Act<T>::load(qkv, (long)b * conv_dim + ch);
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

// grid: (hv * DN_SLICES, batch) workgroups of DN_DEC_NT threads; workgroup
// (h, s) of sequence b owns columns 32 s .. 32 s + 31 of head h (the 4 slices
// of a head on one XCD). Thread t holds rows t / 8 + 32 i (i = 0..3), columns
// 32 s + 4 (t % 8) .. + 3, four 16-byte loads: a wave reads 8 rows' 128-byte
// lines per load. Four waves start together (a larger workgroup's waves start
// in groups of four, about 0.1 us apart).
//
// The arguments are separate scalars, not a struct, so that the first 14
// dwords (the pointers and sizes the first loads need, up to z) are preloaded
// into scalar registers at wave start instead of being read from the argument
// buffer (the library is built with kernel-argument preloading); geo packs
// hv | n_k_heads << 8 | K << 16.
template <typename T>
__global__ __launch_bounds__(DN_DEC_NT) void dn_decode_kernel(
    float* state, const T* qkv, T* ring, const T* conv_w, unsigned geo, unsigned hk_magic, const int* positions,
    const T* z, const float* norm_w, const T* ga, const T* gb, const float* a_neg_p, const float* dt_bias_p, T* out,
    unsigned* sync, float eps) {
  const int hv = geo & 0xff, n_hk = (geo >> 8) & 0xff, K = geo >> 16;
  const int conv_dim = (2 * n_hk + hv) * DN_D;
  const int wg = xcd_remap(blockIdx.x, hv * DN_SLICES);
  const int s = wg & (DN_SLICES - 1), h = wg / DN_SLICES, b = blockIdx.y;
  // h % n_hk without a division: hk_magic = ceil(2^32 / n_hk) is exact for
  // h < 256, but one key head (magic 2^32) does not fit the word
  const int hk = n_hk == 1 ? 0 : h - (int)__umulhi((unsigned)h, hk_magic) * n_hk;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c4 = tid & 7, r = tid >> 3;
  const int col0 = s * DN_DCOLS;
  constexpr int NW = DN_DEC_NT / 64;          // waves: 4
  constexpr int RPT = DN_D * 8 / DN_DEC_NT;   // rows per thread: 4
  constexpr int RSTEP = DN_DEC_NT / 8;        // 32

  QM_PHASE_DECL
  QM_PHASE(0);
  __shared__ float s_q[DN_D], s_k[DN_D], s_v[DN_DCOLS];
  __shared__ float4 s_red[NW][2][DN_DCOLS / 4];   // per wave: the columns' pred and qd partial sums
  __shared__ float4 s_delta[DN_DCOLS / 4];
  __shared__ float s_scal[1];

  // ---- loads, all issued before any is used and none converted before the
  // last is issued: the conv inputs of the head's q and k channels (thread t
  // takes channel t) and of the slice's 32 v channels (wave 0), the state, z,
  // the norm weight of the slice's columns and the head's generation word
  // (wave 0), the position and the gates by scalar loads (uniform).
  const int wv = __builtin_amdgcn_readfirstlane(wid);
  const int key_dim = n_hk * DN_D;
  const int ch_qk = tid < DN_D ? hk * DN_D + tid : key_dim + hk * DN_D + (tid - DN_D);
  const int ch_v = 2 * key_dim + h * DN_D + col0 + (lane & (DN_DCOLS - 1));
  const bool k4 = K == 4;
  ConvIn<T> cin_qk, cin_v;
  if (k4) cin_qk = conv_load4(ring, conv_w, qkv, conv_dim, b, ch_qk);
  // wave 0's v channels ahead of the state, so that their conv waits for
  // nothing else (loads complete in order)
  if (k4 && wv == 0) cin_v = conv_load4(ring, conv_w, qkv, conv_dim, b, ch_v);
  const long head_off = (long)(b * hv + h) * DN_D * DN_D;
  const float4* S = reinterpret_cast<const float4*>(state + head_off) + col0 / 4 + c4;
  float4 st[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) st[i] = S[(r + RSTEP * i) * (DN_D / 4)];
  QM_PHASE(12);
  T zr{};
  float nw = 0.f;
  unsigned* line = sync + (long)(b * hv + h) * DN_SYNC_WORDS;
  unsigned long long* shares = reinterpret_cast<unsigned long long*>(line) + DN_SHARE0;
  unsigned gen = 0;
  if (wv == 0) {
    zr = z[(long)b * hv * DN_D + h * DN_D + col0 + (lane & (DN_DCOLS - 1))];
    nw = norm_w[col0 + (lane & (DN_DCOLS - 1))];
    // the generation word, an atomic load issued last (loads complete in
    // order, so nothing earlier waits for it): it was last written in an
    // earlier launch, and this launch's slice 0 writes it only after every
    // slice of the head has published its share
    gen = ld_flag(line);
  }
  const int pos = uniform_load(positions + b);
  const float gate_b = uniform_act(gb, (long)b * hv + h), gate_a = uniform_act(ga, (long)b * hv + h);
  const float a_neg = uniform_load(a_neg_p + h), dtb = uniform_load(dt_bias_p + h);
  QM_PHASE(6);
  // the decay, in every wave while its conv inputs are in flight
  const float decay = __expf(a_neg * softplus_fast(gate_a + dtb));

  // ---- conv of the q/k channels and the slice's v channels (the q/k ring
  // slots have one writer: slice 0 of the value head h == hk). With K = 4 the
  // ring stores wait for the end: stores and loads share one in-order
  // counter, so a store issued here would hold up the wait for the state.
  const bool qk_writer = h == hk && s == 0;
  // beta = sigmoid(b), rounded to the activation type as the reference rounds
  // it, in wave 1 (a chain of an exponential and a division); it is first
  // needed after the column sums (below), so no barrier waits for it before
  // that.
  float beta_v = 0.f;
  if (tid == 64) beta_v = Act<T>::round(sigmoid_f(gate_b));
  {
    const float y = k4 ? conv_finish4(cin_qk, pos)
                       : conv_channel(ring, conv_w, qkv, conv_dim, K, b, ch_qk, pos, qk_writer);
    if (tid < DN_D) s_q[tid] = y; else s_k[tid - DN_D] = y;
  }
  if (wv == 0) {
    const float y = k4 ? conv_finish4(cin_v, pos)
                       : conv_channel(ring, conv_w, qkv, conv_dim, K, b, ch_v, pos, lane < DN_DCOLS);
    QM_PHASE(7);
    if (lane < DN_DCOLS) s_v[lane] = y;
  }
  __syncthreads();

  QM_PHASE(1);
  // ---- l2 norms of q and k and their dot product, computed by every wave
  // (lane l holds channels l and l + 64): no further barrier
  const float q0 = s_q[lane], q1 = s_q[lane + 64], k0 = s_k[lane], k1 = s_k[lane + 64];
  const float sq = wave_sum(fmaf(q1, q1, q0 * q0));
  const float sk = wave_sum(fmaf(k1, k1, k0 * k0));
  const float sqk = wave_sum(fmaf(q1, k1, q0 * k0));
  // hardware reciprocal square roots and 1/sqrt(d) as a product (about an
  // ulp from the reference's rsqrt and division, far inside the tolerance of
  // the state and outputs)
  const float rq = __builtin_amdgcn_rsqf(sq + 1e-6f), rk = __builtin_amdgcn_rsqf(sk + 1e-6f);
  const float inv_sqrt_d = 0.08838834764831845f;
  const float qk = sqk * rq * rk * inv_sqrt_d;          // q^ . k^
  const float rqd = rq * inv_sqrt_d;                    // q's scale for the four rows

  QM_PHASE(2);
  // ---- per column S^T k^ and S^T q^ of the state before its decay (which
  // scales both sums after they are formed): a thread adds its 4 rows in
  // order, the 8 rows of a wave's load are added across lanes (DPP within
  // rows of 16 lanes, then swaps of row pairs and halves), the 4 waves
  // through LDS
  float kr[RPT];
  float p[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int row = r + RSTEP * i;
    kr[i] = mul_rn(s_k[row], rk);
    const float qr = s_q[row] * rqd;
    p[0] = fmaf(st[i].x, kr[i], p[0]); p[1] = fmaf(st[i].y, kr[i], p[1]);
    p[2] = fmaf(st[i].z, kr[i], p[2]); p[3] = fmaf(st[i].w, kr[i], p[3]);
    p[4] = fmaf(st[i].x, qr, p[4]); p[5] = fmaf(st[i].y, qr, p[5]);
    p[6] = fmaf(st[i].z, qr, p[6]); p[7] = fmaf(st[i].w, qr, p[7]);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = halves_sum(rows_sum(p[i] + dpp_f<0x128>(p[i])));   // row_ror:8
  QM_PHASE(9);
  if (lane < 8) {
    s_red[wid][0][lane] = make_float4(p[0], p[1], p[2], p[3]);
    s_red[wid][1][lane] = make_float4(p[4], p[5], p[6], p[7]);
  }
  if (tid == 64) s_scal[0] = beta_v;
  QM_PHASE(10);
  __syncthreads();

  QM_PHASE(3);
  // ---- delta and o of the 32 columns (wave 0: lanes 0-31 add pred, lanes
  // 32-63 qd, over the 4 waves, then scale them by the decay: pred =
  // (S e^g)^T k^, qd = (S e^g)^T q^), the slice's share of the head's sum of
  // squares of o published with the launch's generation number
  float o = 0.f;
  if (wv == 0) {
    const float* red = reinterpret_cast<const float*>(s_red);
    const int half = lane >> 5, col = lane & (DN_DCOLS - 1);
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) acc += red[(w * 2 + half) * DN_DCOLS + col];
    acc *= decay;
    const float pred = acc, qd = halves_swap(acc);     // lanes 0-31 receive qd
    const float delta = (s_v[col] - pred) * s_scal[0];
    if (lane < DN_DCOLS) reinterpret_cast<float*>(s_delta)[lane] = delta;
    o = lane < DN_DCOLS ? Act<T>::round(fmaf(qk, delta, qd)) : 0.f;
    const float ss = wave_sum(o * o);
    opaque(gen);     // used from here on, not where it is loaded (that would wait for every load there)
    if (lane == 0) {
      const unsigned long long word = ((unsigned long long)(gen + 1) << 32) | __float_as_uint(ss);
      __hip_atomic_store(shares + s, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();

  QM_PHASE(4);
  // ---- decay and rank-1 update (S e^g + k^ delta^T) and write-back of the
  // slice, written through to the point of coherence (no dirty state lines
  // are left in L2 for the end of the kernel), and the deferred ring stores
  {
    const float4 dl = s_delta[c4];
    const __amdgpu_buffer_rsrc_t rsrc = dev_rsrc(state + head_off, DN_D * DN_D * 4);
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      st_dev4(rsrc, ((r + RSTEP * i) * DN_D + col0 + 4 * c4) * 4,
              make_float4(fmaf(kr[i], dl.x, st[i].x * decay), fmaf(kr[i], dl.y, st[i].y * decay),
                          fmaf(kr[i], dl.z, st[i].z * decay), fmaf(kr[i], dl.w, st[i].w * decay)));
  }
  if (k4 && qk_writer) ring[((long)b * conv_dim + ch_qk) * 4 + (pos & 3)] = cin_qk.x;
  if (k4 && wv == 0 && lane < DN_DCOLS) ring[((long)b * conv_dim + ch_v) * 4 + (pos & 3)] = cin_v.x;

  QM_PHASE(5);
  // ---- the head's sum of squares from its 4 shares (one line, polled by
  // wave 0), then the gated RMS norm of the 32 columns
  if (wv == 0) {
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
    QM_PHASE(8);
    if (!done && lane == 0) __hip_atomic_fetch_add(line + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (s == 0 && lane == 0) st_flag(line, gen + 1);
    if (lane < DN_DCOLS) {
      T zv = zr;
      opaque(zv);    // converted here, not where it is loaded (that would wait for the load there)
      // the output is rounded to the activation type: the hardware reciprocal
      // square root and a reciprocal-based sigmoid are well inside that
      const float rn = __builtin_amdgcn_rsqf(ss_all * (1.0f / DN_D) + eps);
      const float y = (nw * (o * rn)) * __builtin_amdgcn_rcpf(1.0f + __expf(-Act<T>::load(&zv, 0)));
      Act<T>::store(out, (long)b * hv * DN_D + h * DN_D + col0 + lane, done ? y : __builtin_nanf(""));
    }
  }
  QM_PHASE(11);
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
  const unsigned geo = (unsigned)g->n_v_heads | ((unsigned)g->n_k_heads << 8) | ((unsigned)g->conv_kernel << 16);
  const unsigned hk_magic = (unsigned)((0x100000000ull + g->n_k_heads - 1) / g->n_k_heads);
  hipLaunchKernelGGL(dn_decode_kernel<T>, dim3(g->n_v_heads * DN_SLICES, g->batch), dim3(DN_DEC_NT), 0, stream,
                     state, static_cast<const T*>(qkv), static_cast<T*>(conv_ring), static_cast<const T*>(conv_w),
                     geo, hk_magic, positions, static_cast<const T*>(z), norm_w, static_cast<const T*>(a),
                     static_cast<const T*>(b), a_neg, dt_bias, static_cast<T*>(out), static_cast<unsigned*>(ws),
                     g->eps);
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
  // one 128-byte line per (sequence, head): generation word, give-up counter
  // and the shares of the gated norm's sum of squares
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
  if (g->n_v_heads > 255 || g->n_k_heads > 255 || g->batch > 65535)
    return qm_fail(QM_ERR_UNSUPPORTED, "qm_dn_decode: n_v_heads and n_k_heads must be below 256, batch below 65536");
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
