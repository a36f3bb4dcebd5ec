// Small HIP runtime shared by the kernels of the quantized matmul path: error
// handling in the reference's style, argument checks, and the operand helpers the
// MFMA kernels share. It takes the place of src/metal_rt.{h,mm} of the reference for
// this path: kernels are compiled offline for gfx950 (template instances instead of
// run-time macro specialisation), buffers are plain device pointers owned by the
// caller, and fatal errors print "raceline: fatal: ..." and exit(1) (metal_rt.mm:16-24).
#pragma once

#include <hip/hip_runtime.h>

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

// ----------------------------------------------------------------- device helpers

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16-bit scale/bias bits -> float, exactly. SD = 0: IEEE half, SD = 1: bfloat16.
template <int SD>
__device__ __forceinline__ float scale_f32(uint16_t bits) {
  if constexpr (SD == 0) {
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
  } else {
    return __uint_as_float(static_cast<uint32_t>(bits) << 16);
  }
}

// Eight 4-bit codes of one uint32 (element e at bits 4e, tools/convert.py:82-89) -> eight
// fp16 operands, in element order. Each half's bit pattern is the code itself, i.e. the
// subnormal q * 2^-24, which is exact; the caller multiplies the scale by 2^24 to undo it.
// Seven VALU ops for eight weights: two masks, one shift, four byte permutes.
__device__ __forceinline__ half8 nib8_to_half8(uint32_t u) {
  const uint32_t lo = u & 0x0F0F0F0Fu;         // bytes: q0 q2 q4 q6
  const uint32_t hi = (u >> 4) & 0x0F0F0F0Fu;  // bytes: q1 q3 q5 q7
  // perm(S0=hi, S1=lo, sel): selector 0..3 picks bytes of lo, 4..7 bytes of hi, 0x0C a zero byte.
  u32x4 d;
  d[0] = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u);  // (q0, q1)
  d[1] = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u);  // (q2, q3)
  d[2] = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u);  // (q4, q5)
  d[3] = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u);  // (q6, q7)
  return __builtin_bit_cast(half8, d);
}

constexpr float kTwo24 = 16777216.0f;  // undoes the 2^-24 of nib8_to_half8

}  // namespace rlq
