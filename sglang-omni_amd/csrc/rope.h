// Rotary position embedding of the code2wav pre-transformer, shared by the rotary kernel of the
// front (code2wav_front.hip) and the qkv GEMM's rotary epilogue (gemm.hip): one definition, so
// both give the same bits (apply_rope_inplace_with_kvcache, sglang_omni/models/qwen3_omni/
// components/code2wav.py:205-215).
#pragma once

#include "common.h"

// A row's start position in its stream: 0 for a first decode (or no slot state), else the
// slot's frame count. Rows whose slot is out of range read position 0 and write no state.
OMNI_DEVICE int64_t row_start(const int64_t* slot_index, const int64_t* positions, int cold,
                              int64_t num_slots, int64_t b, int64_t* slot_out) {
  int64_t slot = -1;
  if (slot_index) {
    slot = slot_index[b];
    if (slot < 0 || slot >= num_slots) slot = -1;
  }
  *slot_out = slot;
  if (cold || !positions || slot < 0) return 0;
  return positions[slot];
}

// sin and cos of a float32 angle (radians) on the hardware v_sin_f32 / v_cos_f32, which take
// revolutions: r = angle / (2 pi) formed as a two-float product with 1 / (2 pi) = kRevHi +
// kRevLo (kRevHi the float nearest, kRevLo the float nearest the rest, together within 7e-17),
// the integer revolutions removed exactly (hi - rint(hi) is exact for |hi| < 2^23), so the
// reduced argument is the float nearest the angle's true fraction of a turn (within 3e-8
// revolutions for the angles position * inv_freq of positions up to 2e5, checked against exact
// arithmetic), however large the angle: a short branch-free sequence in place of the general
// sincosf's range reduction (the qkv GEMM's rotary epilogue measured the same launch time with
// either; its cost is elsewhere).
constexpr float kRevHi = 0.15915493667125702f;
constexpr float kRevLo = 6.4206382432985265e-09f;
OMNI_DEVICE void sincos_rev(float angle, float* s, float* c) {
  // no contraction: hi must be the rounded product (fused into hi - rint(hi), its low part
  // would count twice, once there and once in lo)
#pragma clang fp contract(off)
  const float hi = angle * kRevHi;
  const float lo = __builtin_fmaf(angle, kRevHi, -hi) + angle * kRevLo;
  const float r = (hi - __builtin_rintf(hi)) + lo;
  *s = __builtin_amdgcn_sinf(r);
  *c = __builtin_amdgcn_cosf(r);
}

// The neox pair (x1, x2) = (x[i], x[i + head_dim / 2]) of a head turned by angle
// position * inv_freq[i] (float32): y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin, each one product
// and one fma written out (no contraction left to the compiler), rounded once to bf16.
OMNI_DEVICE void rope_pair(float x1, float x2, float angle, u16* y1, u16* y2) {
#pragma clang fp contract(off)
  float s, c;
  sincos_rev(angle, &s, &c);
  *y1 = float_to_bits_bf16(__builtin_fmaf(x1, c, -(x2 * s)));
  *y2 = float_to_bits_bf16(__builtin_fmaf(x2, c, x1 * s));
}
