// Shared device helpers for the codec decode kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "omni_codec.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16;

#define OMNI_DEVICE __device__ __forceinline__

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Raw buffer access (CDNA buffer resources): a load at an offset outside [0, bytes) returns zeros
// and a store there is dropped, so padding, masked rows and tails need no branches around memory
// instructions (a branch per access would also serialize their completion waits).
constexpr uint32_t kOutOfRange = 0x80000000u;  // every buffer here is smaller than 2 GiB
OMNI_DEVICE __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Round-to-nearest-even float -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
OMNI_DEVICE __bf16 to_bf16(float x) { return (__bf16)x; }
OMNI_DEVICE float from_bf16(__bf16 x) { return (float)x; }

OMNI_DEVICE float bits_to_float_bf16(u16 b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
OMNI_DEVICE u16 float_to_bits_bf16(float x) {
  __bf16 h = to_bf16(x);
  return *reinterpret_cast<u16*>(&h);
}

// IEEE half conversions (round to nearest even) for the fp16 variants of the reference kernels.
OMNI_DEVICE float bits_to_float_f16(u16 b) {
  _Float16 h = *reinterpret_cast<_Float16*>(&b);
  return (float)h;
}
OMNI_DEVICE u16 float_to_bits_f16(float x) {
  _Float16 h = (_Float16)x;
  return *reinterpret_cast<u16*>(&h);
}

// A copy of v the compiler cannot see through. Addresses of rarely run code derived from it are
// computed where they are used instead of being hoisted out of the hot loops and held in
// registers for the whole kernel.
OMNI_DEVICE int opaque_copy(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Snake v + b * sin(2 pi ar v)^2 with the frequency in revolutions, ar = alpha / (2 pi): the
// hardware v_sin_f32 takes revolutions, and v_fract_f32 reduces the phase to [0, 1) (the
// activations are bounded, so no Payne-Hanek style reduction is needed). The kernels stage
// ar = alpha * kInvTwoPi once per coefficient; one expression serves every kernel, so a value
// computed by different kernels rounds alike.
constexpr float kInvTwoPi = 0.15915494309189535f;
OMNI_DEVICE float snake_rev(float v, float ar, float b) {
  const float s = __builtin_amdgcn_sinf(__builtin_amdgcn_fractf(ar * v));
  return v + b * (s * s);
}
// The same with alpha itself (a = alpha, b = 1 / (alpha + 1e-9) for Snake1d).
OMNI_DEVICE float snake_value(float v, float a, float b) { return snake_rev(v, a * kInvTwoPi, b); }

// Activations applied in the conv epilogues.
enum {
  OMNI_ACT_NONE = 0,
  OMNI_ACT_SNAKE = 1,       // x + b * sin(a * x)^2 with per-channel a, b
  OMNI_ACT_LEAKY_RELU = 2,  // x >= 0 ? x : slope * x
  OMNI_ACT_TANH = 3,
  OMNI_ACT_CLAMP = 4,       // clamp(x, -1, 1), NaN propagated
};

// tanh is out of line: inlined at every activation site of an unrolled tile it would multiply
// the kernel's code size, and only the decoder's last layer uses it.
__device__ __noinline__ float act_tanh(float v) { return tanhf(v); }

// The activations applied to conv operands (staging, between fused convs): cheap and inline.
// For Snake, `a` is in revolutions (alpha / (2 pi), see snake_rev).
OMNI_DEVICE float operand_act(int act, float v, float a, float b, float slope) {
  if (act == OMNI_ACT_SNAKE) return snake_rev(v, a, b);
  if (act == OMNI_ACT_LEAKY_RELU) return v >= 0.f ? v : v * slope;
  return v;
}

OMNI_DEVICE float apply_act(int act, float v, float a, float b, float slope) {
  switch (act) {
    case OMNI_ACT_SNAKE:
      return snake_value(v, a, b);
    case OMNI_ACT_LEAKY_RELU:
      return v >= 0.f ? v : v * slope;
    case OMNI_ACT_TANH:
      return act_tanh(v);
    case OMNI_ACT_CLAMP:
      return v != v ? v : fminf(fmaxf(v, -1.f), 1.f);
    default:
      return v;
  }
}

// Workgroup b of a grid of g runs on XCD b % 8 (round-robin dispatch). The logical tile that
// gives XCD x the contiguous range [start(x), start(x + 1)) of tiles, ranges as even as g allows:
// a bijection of [0, g).
constexpr int kNumXcds = 8;
OMNI_DEVICE int xcd_tile(int b, int g) {
  const int xcd = b % kNumXcds;
  const int local = b / kNumXcds;
  const int per = g / kNumXcds;
  const int rem = g % kNumXcds;  // the first rem XCDs take one tile more
  return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

#define OMNI_LAUNCH_CHECK()                                   \
  do {                                                        \
    hipError_t _e = hipGetLastError();                        \
    if (_e != hipSuccess) return OMNI_ERR_LAUNCH;             \
  } while (0)
