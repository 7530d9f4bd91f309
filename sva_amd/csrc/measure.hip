// A plain streaming read of a device buffer: the floor a scan of the same
// bytes is priced against.  Each wave reads 8 KB of consecutive 16-byte
// words (load r of lane l takes word 64 r + l of the wave's span, the code
// scan's own pattern), non-temporal, every load issued before the first is
// used; the words are folded by XOR so the reads cannot be dropped.
#include "capi_internal.h"

namespace {

constexpr int RB = 256;   // threads per workgroup
constexpr int RLPT = 8;   // 16-byte loads per thread
typedef uint32_t u32x4_r __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(RB) stream_read_kernel(const u32x4_r* __restrict__ src, int64_t n16,
                                                         uint32_t* __restrict__ sink) {
  const int64_t wave = (int64_t)blockIdx.x * (RB / 64) + threadIdx.x / 64;
  const int lane = (int)(threadIdx.x & 63);
  const int64_t base = wave * 64 * RLPT;
  u32x4_r v[RLPT];
#pragma unroll
  for (int r = 0; r < RLPT; ++r) {
    const int64_t i = base + r * 64 + lane;
    v[r] = __builtin_nontemporal_load(src + (i < n16 ? i : n16 - 1));  // clamped: every load in bounds
  }
  u32x4_r acc = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int r = 0; r < RLPT; ++r)
    if (base + r * 64 + lane < n16) acc ^= v[r];  // each word once
  sink[(int64_t)blockIdx.x * RB + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

int64_t read_blocks(int64_t bytes) {
  const int64_t n16 = bytes / 16;
  const int64_t per_block = (int64_t)RB * RLPT;  // 16-byte words per workgroup
  return (n16 + per_block - 1) / per_block;
}

}  // namespace

extern "C" int64_t sva_stream_read_sink_words(int64_t bytes) {
  return bytes > 0 ? read_blocks(bytes) * RB : 0;
}

extern "C" int sva_stream_read(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_words, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(src && sink, "sva_stream_read: null pointer");
  SVA_REQUIRE(bytes > 0 && bytes % 16 == 0, "sva_stream_read: bytes must be a positive multiple of 16");
  SVA_REQUIRE(((uintptr_t)src & 15u) == 0, "sva_stream_read: the buffer must be 16-byte aligned");
  const int64_t blocks = read_blocks(bytes);
  SVA_REQUIRE(blocks < (1ll << 31), "sva_stream_read: buffer too large");
  SVA_REQUIRE(sink_words >= blocks * RB, "sva_stream_read: the sink needs %lld words, got %lld",
              (long long)(blocks * RB), (long long)sink_words);
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(RB), 0, (hipStream_t)stream,
                     (const u32x4_r*)src, bytes / 16, sink);
  SVA_CHECK_LAUNCH("stream_read_kernel");
  return SVA_OK;
}
