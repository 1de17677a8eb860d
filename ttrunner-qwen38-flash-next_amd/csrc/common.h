// Shared device helpers for the qwen4mix HIP kernels (gfx950 / CDNA4).
//
// Conventions used by every kernel in this library:
//  * activations are either float32 or bfloat16 (ACT_F32 / ACT_BF16); every
//    kernel is instantiated for both and the entry point dispatches on the enum;
//  * wavefronts are 64 lanes; block reductions go through LDS;
//  * arithmetic that must reproduce PyTorch's CPU rounding bit for bit (the QSA
//    indexer path) uses the explicit *_rn helpers below so that the compiler
//    cannot contract a multiply and an add into one FMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define QM_ACT_F32 0
#define QM_ACT_BF16 1

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4_t;

struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Two floats to packed bf16 (a in the low half) with the hardware conversion
// (v_cvt_pk_bf16_f32: round to nearest even; a NaN stays a quiet NaN): one
// instruction where the integer rounding sequence takes six.
typedef float f32x2_cvt_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_cvt_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2_cvt_t{a, b}, bf16x2_cvt_t));
}

// round-to-nearest-even float32 -> bfloat16 (the hardware conversion)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return static_cast<uint16_t>(pack_bf16x2(f, 0.f)); }

// Activation element access: load as float, store with rounding to the type.
template <typename T> struct Act;
template <> struct Act<float> {
  __device__ __forceinline__ static float load(const float* p, long i) { return p[i]; }
  __device__ __forceinline__ static void store(float* p, long i, float v) { p[i] = v; }
  // value after a round trip through the activation dtype
  __device__ __forceinline__ static float round(float v) { return v; }
};
template <> struct Act<bf16_t> {
  __device__ __forceinline__ static float load(const bf16_t* p, long i) { return bf16_to_f32(p[i].bits); }
  __device__ __forceinline__ static void store(bf16_t* p, long i, float v) { p[i].bits = f32_to_bf16(v); }
  __device__ __forceinline__ static float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};

// A uniform value read through the constant address space, which the compiler
// serves with a scalar load (for buffers the launch does not write, or words
// it writes only after the read).
typedef const float __attribute__((address_space(4)))* cfloat_ptr;
typedef const int __attribute__((address_space(4)))* cint_ptr;
typedef const unsigned __attribute__((address_space(4)))* cu32_ptr;
__device__ __forceinline__ float uniform_load(const float* p) { return *(cfloat_ptr)p; }
__device__ __forceinline__ int uniform_load(const int* p) { return *(cint_ptr)p; }
__device__ __forceinline__ unsigned uniform_load(const unsigned* p) { return *(cu32_ptr)p; }
// element i of an activation buffer at a uniform index; bf16 through the
// aligned 32-bit word that holds it (allocations are 4-byte aligned and
// padded, so the word stays inside the buffer's allocation)
__device__ __forceinline__ float uniform_act(const float* p, long i) { return uniform_load(p + i); }
__device__ __forceinline__ float uniform_act(const bf16_t* p, long i) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(p + i);
  const unsigned w = *(cu32_ptr)(a & ~3ull);
  return bf16_to_f32(static_cast<uint16_t>((a & 2) ? (w >> 16) : (w & 0xffffu)));
}

// Non-contracting float ops: each rounds once, like a CPU SIMD mul/add. hipcc
// compiles with -ffp-contract=fast, and __fmul_rn/__fadd_rn are plain operators,
// so contraction is switched off inside these helpers explicitly: the fmul they
// emit carries no `contract` flag and cannot be fused into a later add.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
// IEEE division and square root (HIP's default for float: correctly rounded)
__device__ __forceinline__ float div_rn(float a, float b) {
#pragma clang fp contract(off)
  return a / b;
}
// correctly rounded 1/sqrt(x), as torch's CPU rsqrt computes it (sqrt, then divide)
__device__ __forceinline__ float rsqrt_rn(float x) { return div_rn(1.0f, __builtin_sqrtf(x)); }

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
// torch.nn.functional.softplus (beta 1, threshold 20) in a short chain of
// hardware exponentials and a logarithm, for the DeltaNet log-decay
// g = a softplus(x) (a = -exp(A_log)): e^x as 2^(x log2 e); log1p(t) as the
// series t - t^2/2 + t^3/3 - t^4/4 below t = 2^-5 (truncation below 2e-7
// relative), else as log(1 + t) with 1 + t rounded to float (below 2e-6
// relative, 1e-7 once t is above 1/2). The library chain (three dependent
// precise calls) takes most of a microsecond in one lane; the decay's error
// stays far inside the state's tolerance.
__device__ __forceinline__ float softplus_fast(float x) {
  if (x > 20.0f) return x;
  const float t = __expf(x);
  return t < 0.03125f ? t * (1.0f - t * (0.5f - t * (0.33333334f - t * 0.25f))) : __logf(1.0f + t);
}

// ---------------------------------------------------------------------------
// Hand-off between the workgroups of one launch, on any die. The data crosses
// through device-scope (sc1) accesses: stores write through to the device's
// point of coherence and loads read from it, so publishing needs no L2
// writeback (a release fence walks the die's whole L2) and reading no L2
// invalidate. A workgroup waits until its own stores have completed before it
// raises its flag; a reader polls the flags, then loads.
//
// Flags carry a generation number: every workgroup of a group reads the
// group's generation word at its start, raises its flag to generation + 1,
// and one workgroup advances the word once every flag has been seen, by which
// time every workgroup of the group has read it. Flags and words start at
// zero (a zeroed workspace); a later launch over fewer workgroups leaves the
// rest of the flags behind, which the wrapping comparison tolerates.
// ---------------------------------------------------------------------------
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
constexpr int CPOL_DEVICE = 16;             // sc1: device-scope coherence
constexpr int BUF_DWORD3 = 0x00020000;      // raw 32-bit buffer resource, gfx9 encoding
constexpr int FLAG_SPIN_MAX = 1 << 20;      // polls before a wait gives up (about a second)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* base, long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, BUF_DWORD3);
}
__device__ __forceinline__ float ld_dev(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, CPOL_DEVICE));
}
__device__ __forceinline__ float ld_dev_bf16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, byte_off, 0, CPOL_DEVICE));
}
__device__ __forceinline__ void st_dev_u32x2(__amdgpu_buffer_rsrc_t r, int byte_off, unsigned lo, unsigned hi) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{lo, hi}, r, byte_off, 0, CPOL_DEVICE);
}
__device__ __forceinline__ float2 ld_dev2(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, CPOL_DEVICE));
}
__device__ __forceinline__ u32x4_t ld_dev_u32x4(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, CPOL_DEVICE));
}
__device__ __forceinline__ void st_dev(__amdgpu_buffer_rsrc_t r, int byte_off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, byte_off, 0, CPOL_DEVICE);
}
__device__ __forceinline__ void st_dev2(__amdgpu_buffer_rsrc_t r, int byte_off, float2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, byte_off, 0, CPOL_DEVICE);
}
__device__ __forceinline__ void st_dev4(__amdgpu_buffer_rsrc_t r, int byte_off, float4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, byte_off, 0, CPOL_DEVICE);
}
__device__ __forceinline__ unsigned ld_flag(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_flag(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Raise a flag (or publish a 64-bit word) by an atomic exchange and wait for
// its return: once it returns the value sits at the point of coherence, so a
// poller's next load sees it (a plain write-through store gets there about
// 300 ns later). The empty asm consumes the old value, which keeps the
// returning form of the atomic.
__device__ __forceinline__ void raise_flag(unsigned* p, unsigned v) {
  const unsigned old = __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::"v"(old));
}
// The same atomic, not waited for: the flag reaches the point of coherence as
// soon, while the wave goes on (its own later loads of the flag see it).
__device__ __forceinline__ void post_flag(unsigned* p, unsigned v) {
  (void)__hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_word(unsigned long long* p, unsigned long long v) {
  const unsigned long long old = __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::"v"(old));
}
// every outstanding memory operation of this wave complete (stores acknowledged)
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }
// One wave polls flags[0..n), n <= MAXN, until each has reached `target` (a
// wrapping comparison); false if it gave up after FLAG_SPIN_MAX polls. A poll
// issues all of a lane's loads before it tests any, so it costs one round trip.
template <int MAXN>
__device__ __forceinline__ bool wait_flags(const unsigned* flags, int n, unsigned target) {
  constexpr int K = (MAXN + 63) / 64;
  const int lane = threadIdx.x & 63;
  for (int it = 0; it < FLAG_SPIN_MAX; ++it) {
    unsigned f[K];
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (64 * k < n) f[k] = ld_flag(flags + min(lane + 64 * k, n - 1));
    bool ok = true;
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (64 * k < n) ok = ok & ((int)(f[k] - target) >= 0);
    if (__builtin_amdgcn_ballot_w64(!ok) == 0ull) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// Workgroups are dealt round-robin to the 8 XCDs; this gives each XCD a
// contiguous range of logical work items so that neighbours share an L2.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  if (n % 8) return bid;
  return (bid % 8) * (n / 8) + bid / 8;
}

// Cross-lane reductions on DPP / readlane / permlane (VALU, a few cycles each)
// rather than __shfl_xor, whose ds_bpermute costs an LDS round trip per step
// and serialises a reduction tree into a chain of LDS latencies.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// sum / max over each row of 16 lanes, result in every lane of the row:
// xor 1, xor 2 (quad_perm), then the half-row and row mirrors
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}
// v(lane) + v(lane ^ 32) and v(lane) + v(lane ^ 16), in every lane (a single
// cross-row step each, so one ds_bpermute is cheap enough)
// the value of lane l ^ 32 / l ^ 16, by v_permlane32_swap / v_permlane16_swap
// of two copies (VALU, no LDS): the 32-lane swap exchanges the upper half of
// one copy with the lower half of the other, the 16-lane swap its odd 16-lane
// rows with the other's even rows
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) { return v + lane_xor32(v); }
__device__ __forceinline__ float xor16_sum(float v) { return v + lane_xor16(v); }
__device__ __forceinline__ float xor32_max(float v) { return fmaxf(v, lane_xor32(v)); }
__device__ __forceinline__ float xor16_max(float v) { return fmaxf(v, lane_xor16(v)); }
// whole-wavefront sum / max, uniform result
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Sum over a block of NT threads (NT a multiple of 64); `red` holds NT/64 floats.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) s += red[i];
  return s;
}

// Sum of squares of `n` floats in LDS, in the order torch's CPU `x.pow(2).mean(-1)`
// reduces a contiguous float32 row: 8-lane vectors into 4 accumulators
// (element e -> accumulator (e/8)%4, lane e%8, in increasing e), the 4
// accumulators added in order lane-wise, then the 8 lanes added in order.
// Requires n % 32 == 0. Called by all threads of the block; thread 0..31 work.
// `scratch` holds 32 floats. Returns the sum (not the mean) in every thread.
__device__ __forceinline__ float torch_row_sumsq(const float* x, int n, float* scratch) {
  const int t = threadIdx.x;
  __syncthreads();
  if (t < 32) {
    float acc = 0.f;
    for (int e = t; e < n; e += 32) acc = add_rn(acc, mul_rn(x[e], x[e]));
    scratch[t] = acc;
  }
  __syncthreads();
  float lanes[8];
#pragma unroll
  for (int l = 0; l < 8; ++l)
    lanes[l] = add_rn(add_rn(add_rn(scratch[l], scratch[8 + l]), scratch[16 + l]), scratch[24 + l]);
  float tot = lanes[0];
#pragma unroll
  for (int l = 1; l < 8; ++l) tot = add_rn(tot, lanes[l]);
  return tot;
}

// Phase markers (a build compiled with -DQM_PHASE_TRACE, for timing a
// kernel's stages; in every other build they are all nothing):
// QM_PHASE_DECL declares a workgroup's 16 LDS time slots; QM_PHASE(slot) has
// thread 0 record the wall clock (100 MHz) in one of them (an LDS write: no
// global store that a later barrier would wait for); QM_PHASE_FLUSH writes the
// slots to the workgroup's row of the translation unit's qm_phase_buf (rows
// from first_row on with QM_PHASE_FLUSH_AT), and
// QM_PHASE_ENTRY(tag) defines qm_phase_read_<tag> / qm_phase_clear_<tag> for
// the host. Slot 15 holds the workgroup's XCC id.
#ifdef QM_PHASE_TRACE
constexpr int QM_PHASE_ROWS = 8192;
static __device__ unsigned long long qm_phase_buf[QM_PHASE_ROWS * 16];
static __shared__ unsigned long long qm_ph_[16];
#define QM_PHASE_DECL \
  if (threadIdx.x < 16) qm_ph_[threadIdx.x] = 0ull;
#define QM_PHASE(slot)                                           \
  do {                                                           \
    if (threadIdx.x == 0) qm_ph_[(slot)] = wall_clock64() | (1ull << 63); \
  } while (0)
#define QM_PHASE_FLUSH() QM_PHASE_FLUSH_AT(0u)
#define QM_PHASE_FLUSH_AT(first_row)                                                                       \
  do {                                                                                                     \
    if (threadIdx.x == 0) {                                                                                \
      const unsigned row_ = (first_row) + blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);  \
      qm_ph_[15] = (unsigned long long)__builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11)) | (1ull << 63); \
      if (row_ < QM_PHASE_ROWS)                                                                            \
        for (int s_ = 0; s_ < 16; ++s_) qm_phase_buf[row_ * 16 + s_] = qm_ph_[s_];                         \
    }                                                                                                      \
  } while (0)
#define QM_PHASE_ENTRY(tag)                                                                              \
  extern "C" int qm_phase_read_##tag(unsigned long long* host, int n) {                                  \
    if (n > QM_PHASE_ROWS * 16) n = QM_PHASE_ROWS * 16;                                                  \
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(qm_phase_buf), n * 8ul) == hipSuccess ? 0 : -1;          \
  }                                                                                                      \
  extern "C" int qm_phase_clear_##tag(void) {                                                            \
    static unsigned long long zeros_[QM_PHASE_ROWS * 16];                                                \
    return hipMemcpyToSymbol(HIP_SYMBOL(qm_phase_buf), zeros_, sizeof(zeros_)) == hipSuccess ? 0 : -1;   \
  }
#else
#define QM_PHASE_DECL
#define QM_PHASE(slot) \
  do {               \
  } while (0)
#define QM_PHASE_FLUSH() \
  do {                 \
  } while (0)
#define QM_PHASE_FLUSH_AT(first_row) \
  do {                             \
  } while (0)
#define QM_PHASE_ENTRY(tag)
#endif

#define QM_CHECK_LAUNCH()                                              \
  do {                                                                 \
    hipError_t e_ = hipGetLastError();                                 \
    if (e_ != hipSuccess) return qm_fail(QM_ERR_LAUNCH, hipGetErrorString(e_)); \
  } while (0)
