// Error state and device queries shared by every C-ABI entry point.
#include <mutex>
#include <vector>

#include "capi_internal.h"
#include "summon.h"

namespace sva {

static thread_local char g_error[1024] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = 0; }

// Compute-unit count of the current device, cached per device ordinal.
int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

}  // namespace sva

extern "C" const char* sva_last_error(void) { return sva::g_error; }

extern "C" int sva_abi_version(void) { return 1; }

namespace {

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

namespace sva {

int fill_u32(uint32_t* ptr, int64_t n, uint32_t value, hipStream_t stream) {
  if (n <= 0) return SVA_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, ptr, n, value);
  SVA_CHECK_LAUNCH("fill_u32_kernel");
  return SVA_OK;
}

int fill_i32(int32_t* ptr, int64_t n, int32_t value, hipStream_t stream) {
  return fill_u32((uint32_t*)ptr, n, (uint32_t)value, stream);
}

}  // namespace sva
