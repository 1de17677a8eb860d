// Device-side services shared by the entry points: the resident capacity of a
// kernel (for launches whose workgroups wait for one another) and a fill kernel
// that clears hand-off words without hipMemsetAsync (a memset node recorded
// into a captured graph is not used anywhere in this library).

#include <atomic>

#include "common.h"
#include "qwen4mix_internal.h"

namespace {

constexpr int MAX_DEVICES = 64;

struct CapacityCache {
  std::atomic<const void*> kernel;
  std::atomic<int> value[MAX_DEVICES];
};

constexpr int MAX_KERNELS = 16;
CapacityCache g_capacity[MAX_KERNELS];
std::atomic<int> g_n_kernels{0};

__global__ void zero_words_kernel(unsigned* p, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace

int qm_resident_workgroups(const void* kernel, int block_threads, size_t dyn_lds, int* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return qm_fail(QM_ERR_LAUNCH, "no current HIP device");
  // one cache slot per kernel, claimed on first use (lookups are lock-free;
  // two threads claiming at once may both compute the same value). A slot's
  // kernel is published with release order after its values are cleared, so
  // a reader that sees the kernel sees cleared or computed values; a slot
  // still being claimed reads as empty (nullptr) and costs a recompute.
  const int n = g_n_kernels.load(std::memory_order_acquire);
  CapacityCache* slot = nullptr;
  for (int i = 0; i < n && i < MAX_KERNELS; ++i)
    if (g_capacity[i].kernel.load(std::memory_order_acquire) == kernel) slot = &g_capacity[i];
  if (slot) {
    const int v = slot->value[dev].load(std::memory_order_relaxed);
    if (v > 0) { *out = v; return QM_OK; }
  }
  int n_cu = 0, per_cu = 0;
  e = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return qm_fail(QM_ERR_LAUNCH, hipGetErrorString(e));
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, dyn_lds);
  if (e != hipSuccess) return qm_fail(QM_ERR_LAUNCH, hipGetErrorString(e));
  const int v = per_cu * n_cu;
  if (!slot) {
    static std::atomic<int> claim{0};
    int mine = claim.fetch_add(1);
    if (mine < MAX_KERNELS) {
      for (int d = 0; d < MAX_DEVICES; ++d) g_capacity[mine].value[d].store(0, std::memory_order_relaxed);
      g_capacity[mine].kernel.store(kernel, std::memory_order_release);
      slot = &g_capacity[mine];
      g_n_kernels.fetch_add(1, std::memory_order_release);
    }
  }
  if (slot) slot->value[dev].store(v, std::memory_order_relaxed);
  *out = v;
  return QM_OK;
}

int qm_zero_words(void* p, long n_words, hipStream_t stream) {
  if (n_words <= 0) return QM_OK;
  const int nt = 256;
  const long nb = (n_words + nt - 1) / nt;
  hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)nb), dim3(nt), 0, stream, static_cast<unsigned*>(p), n_words);
  QM_CHECK_LAUNCH();
  return QM_OK;
}

