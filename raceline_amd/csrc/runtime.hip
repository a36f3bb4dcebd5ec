// Library-level entry points (error mode, last error, device selection) and the runtime
// helpers the kernels' launchers share.
#include "rlq_common.h"
#include "../../include/rlq.h"

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>

namespace rlq {

namespace {
thread_local int t_fatal = 1;
thread_local char t_error[512] = "";
}  // namespace

int fail(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(t_error, sizeof t_error, fmt, ap);
  va_end(ap);
  if (t_fatal) {
    fprintf(stderr, "raceline: fatal: %s\n", t_error);
    fflush(stderr);
    exit(1);
  }
  return -1;
}

int check_hip(hipError_t e, const char *what) {
  if (e == hipSuccess) return 0;
  return fail("%s: %s", what, hipGetErrorString(e));
}

int allow_large_lds(const void *fn, LdsOptIn &done) {
  int dev = 0;
  RLQ_HIP(hipGetDevice(&dev));
  const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && (done.done.load(std::memory_order_acquire) & bit)) return 0;
  RLQ_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLdsBytes));
  if (bit) done.done.fetch_or(bit, std::memory_order_acq_rel);
  return 0;
}

// A plain read stream: every thread loads U 16-byte chunks at once (non-temporal), strided
// by the workgroup so that each load instruction of a wave reads 1 KB contiguous, and folds
// them into an XOR; the store under a condition no real data meets keeps the loads live.
constexpr int kStreamThreads = 512, kStreamUnroll = 8;

__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(const u32x4 *p, size_t n16, float *out) {
  const size_t step = (size_t)gridDim.x * kStreamThreads * kStreamUnroll;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (size_t i = (size_t)blockIdx.x * kStreamThreads * kStreamUnroll + threadIdx.x; i < n16; i += step) {
    u32x4 v[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) {
      const size_t j = i + (size_t)u * kStreamThreads;
      v[u] = j < n16 ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) acc ^= v[u];
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9E3779B9u && acc[0] == 0x7F4A7C15u) out[0] = 1.0f;
}

}  // namespace rlq

extern "C" {

int rlq_abi_version(void) { return 1; }

int rlq_stream_read(const void *p, size_t bytes, float *out, void *stream) {
  RLQ_REQUIRE(p && out && bytes % 16 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0,
              "rlq_stream_read: p and out must be set, p 16-byte aligned, bytes a multiple of 16 (got %zu)", bytes);
  if (bytes == 0) return 0;
  int dev = 0, cus = 0;
  RLQ_HIP(hipGetDevice(&dev));
  RLQ_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const size_t n16 = bytes / 16, per = (size_t)rlq::kStreamThreads * rlq::kStreamUnroll;
  const int blocks = (int)std::min<size_t>((size_t)cus * 4, (n16 + per - 1) / per);
  rlq::stream_read_kernel<<<blocks, rlq::kStreamThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const rlq::u32x4 *>(p), n16, out);
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_set_fatal(int on) {
  int old = rlq::t_fatal;
  rlq::t_fatal = on ? 1 : 0;
  return old;
}

const char *rlq_last_error(void) { return rlq::t_error; }

int rlq_set_device(int device) {
  RLQ_HIP(hipSetDevice(device));
  return 0;
}


}  // extern "C"
