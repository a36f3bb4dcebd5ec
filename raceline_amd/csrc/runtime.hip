// Library-level entry points (error mode, last error, device selection) and the runtime
// helpers the kernels' launchers share.
#include "rlq_common.h"
#include "../../include/rlq.h"

#include <cstdio>
#include <cstdlib>
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

}  // namespace rlq

extern "C" {

int rlq_abi_version(void) { return 1; }

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
