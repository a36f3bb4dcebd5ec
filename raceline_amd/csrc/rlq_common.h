// Small HIP runtime shared by the kernels of the quantized matmul path: error
// handling in the reference's style, argument checks, and the operand helpers the
// MFMA kernels share. It takes the place of src/metal_rt.{h,mm} of the reference for
// this path: kernels are compiled offline for gfx950 (template instances instead of
// run-time macro specialisation), buffers are plain device pointers owned by the
// caller, and fatal errors print "raceline: fatal: ..." and exit(1) (metal_rt.mm:16-24).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
#include <cstdint>

namespace rlq {

// Records an error for the calling thread. In fatal mode (the default) prints it and
// exits with status 1; otherwise returns -1 so the entry point can return it.
int fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
// Checks a HIP status (a launch or a runtime call); returns 0 or fails.
int check_hip(hipError_t e, const char *what);

#define RLQ_REQUIRE(cond, ...)            \
  do {                                    \
    if (!(cond)) return ::rlq::fail(__VA_ARGS__); \
  } while (0)

#define RLQ_HIP(call)                                          \
  do {                                                         \
    int rlq_rc_ = ::rlq::check_hip((call), #call);             \
    if (rlq_rc_) return rlq_rc_;                               \
  } while (0)

inline bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

constexpr size_t kMaxLdsBytes = 160 * 1024;   // LDS of one gfx950 CU

// Lets a kernel use up to kMaxLdsBytes of dynamic LDS on the current device. A function
// attribute belongs to one device, so every device is set once; `done` is the call site's
// record of the devices already set (bit d: device d; devices past 63 are set every call).
struct LdsOptIn {
  std::atomic<uint64_t> done{0};
};
int allow_large_lds(const void *fn, LdsOptIn &done);

// ----------------------------------------------------------------- device helpers

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// 16-bit scale/bias bits -> float, exactly. SD = 0: IEEE half, SD = 1: bfloat16.
template <int SD>
__device__ __forceinline__ float scale_f32(uint16_t bits) {
  if constexpr (SD == 0) {
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
  } else {
    return __uint_as_float(static_cast<uint32_t>(bits) << 16);
  }
}

// Two fp16 values 1024 + a, 1024 + b (a, b < 1024 integers, as the low bits of each half
// over the exponent pattern 0x6400) minus (1024 + OFF): exactly a - OFF and b - OFF, as
// normal fp16 numbers. (Codes go to the matrix cores as normal numbers: the f16 MFMA of
// gfx950 sums products of subnormal operands with about five bits less precision than
// normal ones.)
template <int OFF = 0>
__device__ __forceinline__ uint32_t magic_pair_to_f16(uint32_t bits) {
  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  const half2v m = {(_Float16)(-1024.0f - OFF), (_Float16)(-1024.0f - OFF)};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, bits | 0x64006400u) + m);
}

// Eight 4-bit codes of one uint32 (element e at bits 4e, tools/convert.py:82-89) -> eight
// fp16 operands q0 - OFF .. q7 - OFF, in element order: two masks, one shift, four byte
// permutes, four or + packed-add pairs.
template <int OFF = 0>
__device__ __forceinline__ half8 nib8_to_half8(uint32_t u) {
  const uint32_t lo = u & 0x0F0F0F0Fu;         // bytes: q0 q2 q4 q6
  const uint32_t hi = (u >> 4) & 0x0F0F0F0Fu;  // bytes: q1 q3 q5 q7
  // perm(S0=hi, S1=lo, sel): selector 0..3 picks bytes of lo, 4..7 bytes of hi, 0x0C a zero byte.
  u32x4 d;
  d[0] = magic_pair_to_f16<OFF>(__builtin_amdgcn_perm(hi, lo, 0x0C040C00u));  // (q0, q1)
  d[1] = magic_pair_to_f16<OFF>(__builtin_amdgcn_perm(hi, lo, 0x0C050C01u));  // (q2, q3)
  d[2] = magic_pair_to_f16<OFF>(__builtin_amdgcn_perm(hi, lo, 0x0C060C02u));  // (q4, q5)
  d[3] = magic_pair_to_f16<OFF>(__builtin_amdgcn_perm(hi, lo, 0x0C070C03u));  // (q6, q7)
  return __builtin_bit_cast(half8, d);
}

// Codebooks of the native format (tools/quantlib.py:23-28). kInt15: two's complement
// -8 .. 7; kInt16: the same plus 0.5 (applied as 0.5 * sum of the activations, as
// kernels/linear.metal:128-129,171-172 do); kFp4: e2m1, sign in bit 3.
enum Book { kAffine = 0, kInt15 = 1, kInt16 = 2, kFp4 = 3 };

// Eight native codes -> their codebook values as fp16, in element order.
template <int BOOK>
__device__ __forceinline__ half8 native8_to_half8(uint32_t u) {
  if constexpr (BOOK == kFp4) {
    // magnitude index 0..7 -> high byte of its fp16 value through a byte table (v_perm
    // picks from 8 bytes): 0, 0.5, 1, 1.5, 2, 3, 4, 6 = 0x00, 0x38, 0x3C, 0x3E, 0x40, 0x42, 0x44, 0x46
    constexpr uint32_t kLutLo = 0x3E3C3800u, kLutHi = 0x46444240u;
    const uint32_t mlo = u & 0x07070707u, mhi = (u >> 4) & 0x07070707u;
    const uint32_t slo = u & 0x08080808u, shi = (u >> 4) & 0x08080808u;
    u32x4 d;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t pick = 0x040C000Cu + 0x01000100u * i;            // bytes [0, m(2i), 0, m(2i+1)]
      const uint32_t sel = __builtin_amdgcn_perm(mhi, mlo, pick) | 0x000C000Cu;
      const uint32_t mag = __builtin_amdgcn_perm(kLutHi, kLutLo, sel);
      const uint32_t sgn = __builtin_amdgcn_perm(shi, slo, pick) << 4;  // bit 3 of each code -> bit 15
      d[i] = mag | sgn;
    }
    return __builtin_bit_cast(half8, d);
  } else {
    return nib8_to_half8<8>(u ^ 0x88888888u);   // (q ^ 8) - 8: the signed value
  }
}

}  // namespace rlq
