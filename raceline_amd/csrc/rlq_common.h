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

// Eight native codes -> their codebook values as fp16, in element order. kFp4: the
// hardware's e2m1 -> fp16 conversion, two codes (one byte, low nibble first) per
// instruction; with scale 1 every value is exact: 0, 0.5, 1, 1.5, 2, 3, 4, 6, signed by
// bit 3 (the same bits as a table lookup of the codebook).
template <int BOOK>
__device__ __forceinline__ half8 native8_to_half8(uint32_t u) {
  if constexpr (BOOK == kFp4) {
    u32x4 d;
    d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1.0f, 0));
    d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1.0f, 1));
    d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1.0f, 2));
    d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1.0f, 3));
    return __builtin_bit_cast(half8, d);
  } else {
    return nib8_to_half8<8>(u ^ 0x88888888u);   // (q ^ 8) - 8: the signed value
  }
}

// Eight native codes -> matrix-core operands in the order the tile kernels feed them:
// kFp4 in element order (native8_to_half8); kInt15 and kInt16 in the permuted order
// (q0, q4, q1, q5, q2, q6, q3, q7) of the affine path, which needs no byte permutes: with
// q' = q ^ 8, a mask puts codes 0 and 4 (2 and 6 after a shift by 8) in the mantissas of
// two normal fp16 numbers over the exponent pattern 0x6400, as 1024 + q', and codes 1 and 5
// (3 and 7) as 1024 + 16 q'; one packed add, or fused multiply-add, per pair then gives
// q' - 8, the signed value, exactly: (1024 + q') - 1032 and (1024 + 16 q') / 16 - 72. Ten
// operations for eight codes, against sixteen in element order.
template <int BOOK>
__device__ __forceinline__ half8 native8_operand(uint32_t u) {
  if constexpr (BOOK == kFp4) {
    return native8_to_half8<kFp4>(u);
  } else {
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    const uint32_t v = u ^ 0x88888888u, t = v >> 8;
    const half2v off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const half2v sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f}, off16 = {(_Float16)-72.0f, (_Float16)-72.0f};
    auto lo = [&](uint32_t w) {
      return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, (w & 0x000F000Fu) | 0x64006400u) + off);
    };
    auto hi = [&](uint32_t w) {
      return __builtin_bit_cast(uint32_t,
                                __builtin_bit_cast(half2v, (w & 0x00F000F0u) | 0x64006400u) * sixteenth + off16);
    };
    const u32x4 d = {lo(v), hi(v), lo(t), hi(t)};
    return __builtin_bit_cast(half8, d);
  }
}

}  // namespace rlq
