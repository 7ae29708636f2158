// Fused polyphase convolution on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16).
//
//   acc[b, i, n] = sum_{j < taps} sum_{ci} W[n, j, ci] * u[b, i + j*dil - left_pad, ci]
//
// is an implicit GEMM with the output columns n as the MFMA M dimension, positions as the N
// dimension and (tap, ci) as K. The batch rows form one position space m = b * length + i, so a
// workgroup's tile of BP positions may span several rows (streaming chunks are 12..96 positions
// long): each row segment of the tile is staged with its own (taps-1)*dil halo, and a lane's LDS
// row for position m at tap j is (m - m0) + segment(m) * halo + j * dil. One workgroup owns
// BCO columns x BP positions; per 32-channel K chunk it stages
//   * the tile's input rows (positions plus halos) x 32 channels once in LDS, every tap reading
//     them shifted by j*dil rows, the input activation (Snake / LeakyReLU) applied on the way
//     from float32 or bf16 to the bf16 operand, and
//   * the weights [taps][BCO][32] in LDS,
// both as 64-byte rows, which the 16-row x 4-slot operand reads of the MFMA hit without bank
// conflicts. The next chunk's global loads are issued into registers before the current chunk's
// MFMAs, so memory latency hides behind the matrix cores.
//
// A second, k = 1 conv can be fused behind the first (the residual unit's conv7 -> Snake ->
// conv1): the first GEMM's accumulators go through bias and the middle activation into a bf16
// tile h in LDS, the second GEMM multiplies it by W2 (prefetched into registers during the
// first GEMM's last chunk), and only its result leaves the workgroup.
//
// The epilogue works on the MFMA accumulator layout (lane = position, 4 consecutive channels per
// lane) and fuses the per-column weight scale (fp8), bias, the residual add (in float32, the
// stream read as float32 or float16), the residual-stream store (float32, or float16 rounded to
// nearest even) and the activation (Snake / LeakyReLU / tanh / clamp) into the stores.
//
// Streaming: positions left of 0 come from the slot's history copy (slot_parity & 1); the
// workgroups of column tile 0 write the last left_pad activated input samples into the other
// copy while they stage them, so no separate exchange launch is needed.
#pragma once

#include <type_traits>

#include "common.h"

namespace omni_conv {

constexpr int kChunk = 32;  // input channels per K chunk (one MFMA K step), one 64-byte LDS row
constexpr int kMaxHalo = 64;

struct ConvParams {
  const void* x;
  int64_t x_sb, x_st;
  int batch, length, c_in, x_length;
  int in_act;
  const float* in_a;
  const float* in_b;
  float in_slope;
  const void* weight;
  const float* wscale;
  int n_cols, c_out, taps, dil, lpad, halo;
  const float* bias;
  const void* weight2;
  const float* wscale2;
  const float* bias2;
  int mid_act;
  const float* mid_a;
  const float* mid_b;
  float mid_slope;
  const u16* hist;  // pool base, NULL if no history
  const int64_t* slot_index;
  const int64_t* slot_parity;
  int64_t hist_slots;
  int64_t hist_slot_stride;
  int hist_cold;
  const void* residual;  // float32, or float16 when r_f16
  int64_t r_sb, r_st;  // shared by residual, mix_a, mix_b and sum_out
  const void* mix_a;  // float32, or float16 with r_f16
  const void* mix_b;
  void* sum_out;  // float32, or float16 when r_f16
  int r_f16;      // residual, mix and sum_out are float16 (a half-precision residual stream)
  void* out;
  int out_bf16;
  int64_t o_sb, o_st;
  int act;
  const float* act_a;
  const float* act_b;
  float slope;
  float mix_scale;
  int p_tiles, n_tiles;
  // split-K (LDS-DMA k = 1 convs only): k_splits slices of whole 32-channel chunks, slice s
  // writing its float32 partial tile [positions][n_cols] at partial + s * positions * n_cols
  int k_splits;
  float* partial;
  // byte extents of the buffers the kernel reads and writes (each below 2 GiB)
  uint32_t x_bytes, w_bytes, w2_bytes, hist_bytes, r_bytes, o_bytes;
};

// Two floats to a bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}

// Eight OCP e4m3fn bytes -> eight bf16, byte i to element i (exact: every e4m3fn value, the
// subnormals included, is a bf16 value; 0x7f / 0xff are NaN). gfx950 converts a byte pair per
// v_cvt_scalef32_pk_bf16_fp8 (scale 1; word_sel picks bytes 0-1 or 2-3 of the dword).
template <bool HIGH>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t word) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, HIGH));
}
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(u32x2 raw) {
  return u32x4{fp8x2_to_bf16x2<false>(raw[0]), fp8x2_to_bf16x2<true>(raw[0]),
               fp8x2_to_bf16x2<false>(raw[1]), fp8x2_to_bf16x2<true>(raw[1])};
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_ROWS, int MAX_TAPS>
struct ConvTile {
  static constexpr int NT = 64 * WAVES_CO * WAVES_P;
  static constexpr int BCO = WAVES_CO * TCO * 16;
  static constexpr int BP = WAVES_P * TP * 16;
  static constexpr int X_PIECES = (MAX_ROWS * 4 + NT - 1) / NT;
  static constexpr int W_PIECES = (BCO * MAX_TAPS * 4 + NT - 1) / NT;
  static_assert(W_PIECES <= 32 && X_PIECES <= 16, "per-thread piece masks are 32-bit");
  // Weights in LDS: one row per output column holding its taps x 32 channels, padded by 32 bytes
  // to a pitch of 2 mod 4 16-byte slots, at which the 16 rows an operand read touches meet no
  // LDS bank conflict.
  static constexpr int64_t wrow(int64_t taps) { return taps * kChunk + 16; }
  // Epilogue: the accumulator tile goes through LDS as float32 rows of BCO (+ 4 pad) columns,
  // half the position waves at a time, so the stores to HBM are whole contiguous rows.
  static constexpr int EPITCH = BCO + 4;
  static constexpr int EPI_ROWS = ((WAVES_P + 1) / 2) * TP * 16;
  // LDS bytes: the first GEMM's staging, the fused second GEMM's h tile and W2, or the epilogue
  static constexpr size_t lds_bytes(int64_t rows, int64_t taps, bool fuse2) {
    const size_t first = (size_t)rows * kChunk * 2 + (size_t)BCO * wrow(taps) * 2;
    const size_t second = fuse2 ? (size_t)BCO * (BP + BCO) * 2 : 0;
    const size_t epi = (size_t)EPI_ROWS * EPITCH * 4;
    const size_t m = first > second ? first : second;
    return (m > epi ? m : epi) + coef_bytes();
  }
  // Per-column epilogue coefficients, staged once per workgroup at the end of LDS: rows
  // scale, bias, mid_a, mid_b, scale2, bias2, act_a, act_b of BCO floats each (the Snake
  // frequencies mid_a and act_a in revolutions).
  static constexpr int NCOEF = 8;  // kNumCoefRows
  static constexpr size_t coef_bytes() { return (size_t)NCOEF * BCO * 4; }
  static constexpr size_t coef_offset(int64_t rows, int64_t taps, bool fuse2) {
    return lds_bytes(rows, taps, fuse2) - coef_bytes();
  }
};

// The activation the staging applies to an input element of channel c.
__device__ __forceinline__ float in_activation(int act, float v, float a, float b, float slope) {
  return operand_act(act, v, a, b, slope);
}

// Rows of the per-column epilogue coefficient table (ConvTile::NCOEF rows of BCO floats).
enum CoefRow { kScale, kBias, kMidA, kMidB, kScale2, kBias2, kActA, kActB, kNumCoefRows };

// The epilogue's per-column coefficients of column tile n0 into LDS (visible after the caller's
// next barrier): the fp8 weight scale, bias, the fused k = 1 conv's middle Snake, scale and bias,
// and the output activation's coefficients (Snake frequencies in revolutions).
template <int BCO, int NT, bool FUSE2>
__device__ __forceinline__ void stage_coefficients(const ConvParams& p, float* coef, int n0) {
  const int tid = threadIdx.x;
  const int n_cols = p.n_cols;
  for (int e = tid; e < kNumCoefRows * BCO; e += NT) {
    const int k = e / BCO;
    const int j = e - k * BCO;
    const int n = n0 + j;
    const bool real = n < n_cols;
    const int co = real ? n % p.c_out : 0;
    float v = (k == kScale || k == kScale2) ? 1.f : 0.f;
    if (real) {
      switch (k) {
        case kScale: if (p.wscale) v = p.wscale[n]; break;
        case kBias: if (p.bias) v = p.bias[co]; break;
        case kMidA: if (FUSE2 && p.mid_a) v = p.mid_a[co] * kInvTwoPi; break;
        case kMidB: if (FUSE2 && p.mid_b) v = p.mid_b[co]; break;
        case kScale2: if (FUSE2 && p.wscale2) v = p.wscale2[n]; break;
        case kBias2: if (FUSE2 && p.bias2) v = p.bias2[co]; break;
        case kActA: if (p.act_a) v = p.act_a[co] * kInvTwoPi; break;
        default: if (p.act_b) v = p.act_b[co]; break;
      }
    }
    coef[e] = v;
  }
}

// Four consecutive elements of a residual stream at byte offset off (kOutOfRange reads zeros),
// as loaded: float32 (one 16-byte load), or float16 (one 8-byte load, in the first two words).
// The raw bits are widened only where they are used (widen_residual4), so a prefetch's wait stays
// at its use.
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 load_residual4_raw(__amdgpu_buffer_rsrc_t rsrc, uint32_t off,
                                                    int f16) {
  if (f16) {
    const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rsrc, off, 0, 0);
    return u32x4{w.x, w.y, 0u, 0u};
  }
  return __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
}
// The four float32 values of a raw residual load (float16 widened exactly).
__device__ __forceinline__ f32x4 widen_residual4(u32x4 raw, int f16) {
  if (f16) return __builtin_convertvector(__builtin_bit_cast(f16x4, u32x2{raw.x, raw.y}), f32x4);
  return __builtin_bit_cast(f32x4, raw);
}
__device__ __forceinline__ f32x4 load_residual4(__amdgpu_buffer_rsrc_t rsrc, uint32_t off,
                                                int f16) {
  return widen_residual4(load_residual4_raw(rsrc, off, f16), f16);
}
// ... and the store: float32, or float16 rounded to nearest even (kOutOfRange drops it).
__device__ __forceinline__ void store_residual4(f32x4 v, __amdgpu_buffer_rsrc_t rsrc, uint32_t off,
                                                int f16) {
  if (f16)
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, __builtin_convertvector(v, f16x4)),
                                          rsrc, off, 0, 0);
  else
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rsrc, off, 0, 0);
}

// The epilogue shared by the conv kernels, from the accumulators of a BCO x BP tile (column
// tile n0, positions [m0, m_end)) to HBM, in two steps per pass over half the position waves:
// (1) in the accumulator layout (lane = position, 4 consecutive columns per lane) each wave adds
// the weight scale and bias and writes float32 rows into LDS; (2) the workgroup walks those rows
// 16 bytes per thread, so the residual / mix loads and the sum_out / out stores are whole
// contiguous rows of HBM. `lds` must be free for Tile::EPI_ROWS x Tile::EPITCH floats (the first
// pass begins with a barrier); `coef` holds the tile's coefficient table. MIX = false: a kernel
// whose launcher refuses the mix leaves out its code (and the registers it takes).
template <typename Tile, int WAVES_P, int TCO, int TP, bool MIX, bool F16>
__device__ __forceinline__ void conv_epilogue_body(const ConvParams& p, f32x4 (&acc)[TCO][TP], u16* lds,
                                              const float* coef, int coef_scale, int coef_bias,
                                              int n0, int m0, int m_end, int wave_p, int wco0) {
  constexpr int NT = Tile::NT;
  constexpr int BCO = Tile::BCO;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int lrow = lane & 15;
  const int ch_in_tile = (lane >> 4) * 4;
  const int L = p.length;
  const int n_cols = p.n_cols;
  constexpr int EPITCH = Tile::EPITCH;
  constexpr int EPI_WAVES = Tile::EPI_ROWS / (TP * 16);  // position waves per pass
  constexpr int QUADS = BCO / 4;                         // 16-byte column groups per row
  constexpr int RSTEP = NT / QUADS;                      // rows a workgroup pass walks at once
  float* ep = reinterpret_cast<float*>(lds);
  // step 2's fixed column group per thread, and its activation coefficients
  const int q = tid % QUADS;
  const int r_first = tid / QUADS;
  const bool walker = r_first < RSTEP;
  const int n_q = n0 + q * 4;
  const f32x4 act_a = *reinterpret_cast<const f32x4*>(coef + kActA * BCO + q * 4);
  const f32x4 act_b = *reinterpret_cast<const f32x4*>(coef + kActB * BCO + q * 4);
  const float inv_l = 1.f / (float)L;
  // Packed tensors (row stride = length x position stride, the decoders' usual layout) address a
  // position by its flat index m alone; otherwise m splits into (row, position). Element offsets
  // fit 32 bits (the byte extents are below 2 GiB).
  const bool packed = p.r_sb == (int64_t)L * p.r_st && p.o_sb == (int64_t)L * p.o_st;
  const uint32_t r_st = (uint32_t)p.r_st, o_st = (uint32_t)p.o_st;
  const uint32_t rsize = F16 ? 2u : 4u;  // bytes per residual-stream element
  const bool live = walker && n_q < n_cols;
  // element offsets of flat position m in the residual-shaped tensors and in out
  // (for NU positions at once: the packed / general choice is one branch for all of them)
  auto offsets = [&](const auto& m, auto& re, auto& oe) __attribute__((always_inline)) {
    constexpr int NU = sizeof(m) / sizeof(m[0]);
    if (packed) {
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        re[u] = (uint32_t)m[u] * r_st + n_q;
        oe[u] = (uint32_t)m[u] * o_st + n_q;
      }
    } else {
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        int b = (int)((float)m[u] * inv_l);  // m / L, corrected below
        int i = m[u] - b * L;
        if (i < 0) { --b; i += L; }
        if (i >= L) { ++b; i -= L; }
        re[u] = (uint32_t)(b * p.r_sb + (int64_t)i * p.r_st + n_q);
        oe[u] = (uint32_t)(b * p.o_sb + (int64_t)i * p.o_st + n_q);
      }
    }
  };
  // Finish the NU rows r0 + u * RSTEP of a pass (positions from mp, prow rows; r0 < prow): read
  // them from LDS, add the residual (`res`, loaded beforehand when `have_res`, else loaded here)
  // and the mix, store sum_out, apply the activation and store out.
  auto finish = [&](auto nu, int mp, int prow, int r0, bool have_res, auto& res)
      __attribute__((always_inline)) {
    constexpr int NU = decltype(nu)::value;
    uint32_t roff[NU], ooff[NU];
    f32x4 v[NU];
    int ms[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) ms[u] = mp + min(r0 + u * RSTEP, prow - 1);
    offsets(ms, roff, ooff);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const bool ok = live && r0 + u * RSTEP < prow;
      roff[u] = ok ? roff[u] * rsize : kOutOfRange;
      ooff[u] = ok ? ooff[u] : kOutOfRange;
      v[u] = *reinterpret_cast<const f32x4*>(ep + (ms[u] - mp) * EPITCH + q * 4);
    }
    if (p.residual) {
      if (!have_res) {
        const auto rr = buffer_rsrc(p.residual, p.r_bytes);
#pragma unroll
        for (int u = 0; u < NU; ++u) res[u] = load_residual4_raw(rr, roff[u], F16);
      }
#pragma unroll
      for (int u = 0; u < NU; ++u) v[u] += widen_residual4(res[u], F16);
    }
    if (MIX && p.mix_a) {
      const auto ra = buffer_rsrc(p.mix_a, p.r_bytes);
      const auto rb = buffer_rsrc(p.mix_b, p.r_bytes);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const f32x4 ma = load_residual4(ra, roff[u], F16);
        const f32x4 mb = load_residual4(rb, roff[u], F16);
        v[u] = ((ma + mb) + v[u]) * p.mix_scale;
      }
    }
    if (p.sum_out) {
      const auto rs = buffer_rsrc(p.sum_out, p.r_bytes);
#pragma unroll
      for (int u = 0; u < NU; ++u) store_residual4(v[u], rs, roff[u], F16);
    }
    if (p.out != nullptr) {
      // the activation, then the stores, each branch taken once for the NU rows (a branch per
      // row keeps the compiler from grouping the rows' stores)
      const int act = p.act;
      if (act == OMNI_ACT_SNAKE) {
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[u][e] = snake_rev(v[u][e], act_a[e], act_b[e]);
      } else if (act == OMNI_ACT_LEAKY_RELU) {
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[u][e] = v[u][e] >= 0.f ? v[u][e] : v[u][e] * p.slope;
      } else if (act != OMNI_ACT_NONE) {
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[u][e] = apply_act(act, v[u][e], 0.f, 0.f, p.slope);
      }
      const auto ro = buffer_rsrc(p.out, p.o_bytes);
      if (p.out_bf16) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const uint32_t oo = ooff[u] == kOutOfRange ? kOutOfRange : ooff[u] * 2;
          __builtin_amdgcn_raw_buffer_store_b64(
              u32x2{pack_bf16x2(v[u][0], v[u][1]), pack_bf16x2(v[u][2], v[u][3])}, ro, oo, 0, 0);
        }
      } else {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const uint32_t oo = ooff[u] == kOutOfRange ? kOutOfRange : ooff[u] * 4;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[u]), ro, oo, 0, 0);
        }
      }
    }
  };
  // When a walker's rows of a pass fit in registers (UR of them), the pass's residual rows are
  // loaded before its LDS exchange (the first pass's before the first barrier, a later pass's
  // right after the previous pass's stores were issued): their HBM latency then overlaps the
  // exchange instead of costing a round trip per group of rows after it.
  constexpr int NPASS = (WAVES_P + EPI_WAVES - 1) / EPI_WAVES;
  constexpr int UR = (Tile::EPI_ROWS + RSTEP - 1) / RSTEP;  // rows per walker and pass
  constexpr bool PREFETCH = UR <= 10 && NT <= 512;
  u32x4 pre[PREFETCH ? UR : 1];  // raw residual loads (load_residual4_raw)
  auto prefetch = [&](int pass) __attribute__((always_inline)) {
    if constexpr (PREFETCH) {
      if (p.residual) {
        const auto rr = buffer_rsrc(p.residual, p.r_bytes);
        const int mp = m0 + pass * Tile::EPI_ROWS;
        const int prow = min(Tile::EPI_ROWS, m_end - mp);
        int ms[UR];
        uint32_t re[UR], oe[UR];
#pragma unroll
        for (int u = 0; u < UR; ++u) ms[u] = mp + min(r_first + u * RSTEP, prow - 1);
        offsets(ms, re, oe);
#pragma unroll
        for (int u = 0; u < UR; ++u) {
          const uint32_t off = live && r_first + u * RSTEP < prow ? re[u] * rsize : kOutOfRange;
          pre[u] = load_residual4_raw(rr, off, F16);
        }
      }
    }
  };
  prefetch(0);
#pragma unroll
  for (int pass = 0; pass < NPASS; ++pass) {
    if (pass > 0) prefetch(pass);
    __syncthreads();
    const int wl = wave_p - pass * EPI_WAVES;  // this wave's slot in the pass
    if (wl >= 0 && wl < EPI_WAVES) {
#pragma unroll
      for (int c = 0; c < TCO; ++c) {
        const int col = wco0 + c * 16 + ch_in_tile;
        const f32x4 sc = *reinterpret_cast<const f32x4*>(coef + coef_scale * BCO + col);
        const f32x4 bi = *reinterpret_cast<const f32x4*>(coef + coef_bias * BCO + col);
#pragma unroll
        for (int t = 0; t < TP; ++t) {
          float* row = ep + (wl * TP * 16 + t * 16 + lrow) * EPITCH + col;
          *reinterpret_cast<f32x4*>(row) = acc[c][t] * sc + bi;
        }
      }
    }
    __syncthreads();
    const int mp = m0 + pass * Tile::EPI_ROWS;  // first position of the pass
    const int prow = min(Tile::EPI_ROWS, m_end - mp);
    if constexpr (PREFETCH) {
      if (r_first < prow) finish(std::integral_constant<int, UR>{}, mp, prow, r_first, true, pre);
    } else {
      constexpr int U = 4;  // rows in flight per thread
      for (int r0 = r_first; r0 < prow; r0 += U * RSTEP) {
        u32x4 res[U];
        finish(std::integral_constant<int, U>{}, mp, prow, r0, false, res);
      }
    }
  }
}

// The residual stream's dtype is a compile-time constant of each copy of the epilogue, so its
// loads, stores and widening take no per-row select.
template <typename Tile, int WAVES_P, int TCO, int TP, bool MIX = true>
__device__ __forceinline__ void conv_epilogue(const ConvParams& p, f32x4 (&acc)[TCO][TP], u16* lds,
                                              const float* coef, int coef_scale, int coef_bias,
                                              int n0, int m0, int m_end, int wave_p, int wco0) {
  if (p.r_f16)
    conv_epilogue_body<Tile, WAVES_P, TCO, TP, MIX, true>(p, acc, lds, coef, coef_scale, coef_bias,
                                                          n0, m0, m_end, wave_p, wco0);
  else
    conv_epilogue_body<Tile, WAVES_P, TCO, TP, MIX, false>(p, acc, lds, coef, coef_scale,
                                                           coef_bias, n0, m0, m_end, wave_p, wco0);
}

// Input modes: bf16 used as is; bf16 activated while staged; float32 activated while staged.
enum { IN_RAW = 0, IN_ACT = 1, IN_F32 = 2 };

template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_ROWS, int MAX_TAPS, int IN,
          bool W_FP8, bool FUSE2>
__global__ void __launch_bounds__(64 * WAVES_CO * WAVES_P)
    conv_mfma_kernel(const ConvParams p) {
  using Tile = ConvTile<WAVES_CO, WAVES_P, TCO, TP, MAX_ROWS, MAX_TAPS>;
  constexpr int NT = Tile::NT;
  constexpr int BCO = Tile::BCO;
  constexpr int BP = Tile::BP;
  extern __shared__ __attribute__((aligned(16))) u16 lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_co = wave % WAVES_CO;
  const int wave_p = wave / WAVES_CO;

  // blockIdx -> (position tile, column tile), numbered per XCD (xcd_tile) with the column tile
  // fastest, so the workgroups that share an input tile run back to back on one XCD.
  const int n_tile = xcd_tile(blockIdx.x, gridDim.x) % p.n_tiles;
  const int p_tile = xcd_tile(blockIdx.x, gridDim.x) / p.n_tiles;
  const int n0 = n_tile * BCO;

  const int taps = p.taps;
  const int dil = p.dil;
  const int lpad = p.lpad;
  const int halo = p.halo;
  const int L = p.length;     // output positions per row
  const int XL = p.x_length;  // input positions per row (the history ends at XL)
  const int H = lpad;         // history samples when streaming
  const int c_in = p.c_in;
  const int n_cols = p.n_cols;

  // The tile's positions [m0, m_end) of the flattened (row, position) space and its row segments.
  const int M = p.batch * L;
  const int m0 = p_tile * BP;
  const int m_end = min(m0 + BP, M);
  const int b0 = m0 / L;
  const int lo0 = m0 - b0 * L;
  const int first = min(L - lo0, m_end - m0);  // tile positions in row b0
  const int nseg = (m_end - 1) / L - b0 + 1;
  const int rows = (m_end - m0) + nseg * halo;  // staged input rows
  const int seg_rows = L + halo;                // staged rows of a full later segment

  u16* xs = lds;                        // [rows][32]
  u16* ws = lds + MAX_ROWS * kChunk;    // [BCO][taps * 32 + 8]
  const int WROW = (int)Tile::wrow(taps);

  const int chunks = (c_in + kChunk - 1) / kChunk;
  const int q8 = (tid & 3) * 8;  // NT is a multiple of 4: a thread stages the same quarter of every row

  // Per-thread staging descriptors, computed once: each input piece's element offset at channel
  // q8 of chunk 0 (in x, or in the history pool), its source (2 bits: 0 zeros, 1 x, 2 history)
  // and, when it is a sample of the new history this workgroup writes, its offset there.
  int xoff[Tile::X_PIECES];
  int hwoff[Tile::X_PIECES];
  unsigned xmode = 0;
  const bool may_write_history = p.hist != nullptr && n_tile == 0 && H > 0;
#pragma unroll
  for (int u = 0; u < Tile::X_PIECES; ++u) {
    const int r = (tid >> 2) + u * (NT / 4);
    int off = 0;
    int hw = -1;
    if (r < rows) {
      int b, pos;
      bool row_start;  // the tile holds position 0 of row b
      if (r < first + halo) {
        b = b0;
        pos = lo0 - lpad + r;
        row_start = lo0 == 0;
      } else {
        const int rr = r - (first + halo);
        const int s = rr / seg_rows;
        b = b0 + 1 + s;
        pos = rr - s * seg_rows - lpad;
        row_start = true;
      }
      int64_t slot = -1;
      int64_t parity = 0;
      if (p.hist != nullptr) {
        slot = p.slot_index[b];
        if (slot >= p.hist_slots) slot = -1;
        if (slot >= 0) parity = p.slot_parity[slot] & 1;
      }
      if (pos >= 0 && pos < XL) {
        off = (int)(b * p.x_sb + (int64_t)pos * p.x_st) + q8;
        xmode |= 1u << (2 * u);
      } else if (pos < 0 && slot >= 0 && !p.hist_cold) {
        off = (int)(slot * p.hist_slot_stride + (parity * H + (H + pos)) * (int64_t)c_in) + q8;
        xmode |= 2u << (2 * u);
      }
      if (may_write_history && slot >= 0 && pos >= XL - H && pos < XL) {
        // each sample of the new history is written by the workgroup whose tile holds it (the
        // samples left of 0 by the one holding position 0)
        const int64_t m = (int64_t)b * L + pos;
        const bool owned = pos >= 0 ? (m >= m0 && m < m_end) : row_start;
        if (owned)
          hw = (int)(slot * p.hist_slot_stride + ((1 - parity) * H + (pos - (XL - H))) *
                                                     (int64_t)c_in) + q8;
      }
    }
    xoff[u] = off;
    hwoff[u] = hw;
  }
  int wlds[Tile::W_PIECES];
  unsigned wreal = 0;
#pragma unroll
  for (int u = 0; u < Tile::W_PIECES; ++u) {
    const int piece = tid + u * NT;
    int off = -1;
    if (piece < BCO * taps * 4) {
      // packed order within a chunk is [n][tap][32]
      const int nl = piece / (taps * 4);
      const int rem = piece - nl * taps * 4;
      off = nl * WROW + (rem >> 2) * kChunk + (rem & 3) * 8;
      if (n0 + nl < n_cols) wreal |= 1u << u;
    }
    wlds[u] = off;
  }

  // Raw 16-byte loads per input piece: 8 float32 (two registers) or 8 bf16 (one) of x, or 8 bf16
  // of history in the first register.
  constexpr bool X_F32 = IN == IN_F32;
  constexpr int XV = X_F32 ? 2 : 1;
  u32x4 xr[Tile::X_PIECES][XV];
  u32x4 wr[W_FP8 ? 1 : Tile::W_PIECES];
  u32x2 wr8[W_FP8 ? Tile::W_PIECES : 1];
  float ina[8], inb[8];

  const u16* hist = p.hist;
  const auto x_rsrc = buffer_rsrc(p.x, p.x_bytes);
  const auto h_rsrc = buffer_rsrc(p.hist, p.hist_bytes);
  const auto w_rsrc = buffer_rsrc(p.weight, p.w_bytes);
  constexpr uint32_t XE = X_F32 ? 4 : 2;  // bytes per x element
  constexpr uint32_t WE = W_FP8 ? 1 : 2;  // bytes per weight element
  auto load_chunk = [&](int kc) __attribute__((always_inline)) {
    const bool in_range = kc * kChunk + q8 < c_in;
#pragma unroll
    for (int u = 0; u < Tile::X_PIECES; ++u) {
      const unsigned mode = (xmode >> (2 * u)) & 3u;
      const uint32_t e = (uint32_t)(xoff[u] + kc * kChunk);
      const uint32_t xo = (mode == 1 && in_range) ? e * XE : kOutOfRange;
      xr[u][0] = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, xo, 0, 0);
      if constexpr (X_F32) xr[u][1] = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, xo + 16, 0, 0);
    }
    if (hist != nullptr) {
      // history rows (bf16, already activated) into the first register of their pieces; the x
      // loads of those pieces were out of range, so they read zeros
#pragma unroll
      for (int u = 0; u < Tile::X_PIECES; ++u) {
        const unsigned mode = (xmode >> (2 * u)) & 3u;
        const uint32_t ho = (mode == 2 && in_range) ? (uint32_t)(xoff[u] + kc * kChunk) * 2
                                                    : kOutOfRange;
        xr[u][0] |= __builtin_amdgcn_raw_buffer_load_b128(h_rsrc, ho, 0, 0);
      }
    }
    if (IN != IN_RAW && p.in_act == OMNI_ACT_SNAKE && in_range) {
      const float4 a0 = *reinterpret_cast<const float4*>(p.in_a + kc * kChunk + q8);
      const float4 a1 = *reinterpret_cast<const float4*>(p.in_a + kc * kChunk + q8 + 4);
      const float4 b0v = *reinterpret_cast<const float4*>(p.in_b + kc * kChunk + q8);
      const float4 b1v = *reinterpret_cast<const float4*>(p.in_b + kc * kChunk + q8 + 4);
      ina[0] = a0.x; ina[1] = a0.y; ina[2] = a0.z; ina[3] = a0.w;
      ina[4] = a1.x; ina[5] = a1.y; ina[6] = a1.z; ina[7] = a1.w;
#pragma unroll
      for (int e = 0; e < 8; ++e) ina[e] *= kInvTwoPi;  // Snake frequency in revolutions
      inb[0] = b0v.x; inb[1] = b0v.y; inb[2] = b0v.z; inb[3] = b0v.w;
      inb[4] = b1v.x; inb[5] = b1v.y; inb[6] = b1v.z; inb[7] = b1v.w;
    }
    const uint32_t wbase = (uint32_t)(((int64_t)kc * n_cols + n0) * taps * kChunk);
#pragma unroll
    for (int u = 0; u < Tile::W_PIECES; ++u) {
      const uint32_t wo = (wreal & (1u << u)) ? (wbase + (uint32_t)(tid + u * NT) * 8) * WE
                                              : kOutOfRange;
      if constexpr (W_FP8) wr8[u] = __builtin_amdgcn_raw_buffer_load_b64(w_rsrc, wo, 0, 0);
      else wr[u] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, wo, 0, 0);
    }
  };

  // W2 (the fused k = 1 conv, [C/32][C][32]) into the weight prefetch registers.
  constexpr int W2_PIECES = FUSE2 ? (BCO * BCO / 8 + NT - 1) / NT : 0;
  static_assert(W2_PIECES <= Tile::W_PIECES, "W2 must fit the weight prefetch registers");
  const auto w2_rsrc = buffer_rsrc(p.weight2, p.w2_bytes);
  auto load_w2 = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < W2_PIECES; ++u) {
      const int piece = tid + u * NT;
      const uint32_t wo = piece < BCO * BCO / 8 ? (uint32_t)piece * 8 * WE : kOutOfRange;
      if constexpr (W_FP8) wr8[u] = __builtin_amdgcn_raw_buffer_load_b64(w2_rsrc, wo, 0, 0);
      else wr[u] = __builtin_amdgcn_raw_buffer_load_b128(w2_rsrc, wo, 0, 0);
    }
  };

  // The bf16 operand of input piece u: x (activated unless IN_RAW), history (already activated)
  // or zeros (padding, channels past c_in: their loads were out of range, and every activation
  // maps 0 to 0). Always inlined: a call would force the register arrays into scratch memory.
  auto stage_value = [&](int u) __attribute__((always_inline)) -> u32x4 {
    if constexpr (IN == IN_RAW) {
      return xr[u][0];
    } else {
      const bool is_hist = ((xmode >> (2 * u)) & 3u) == 2u;
      float v[8];
      if constexpr (X_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = __uint_as_float(xr[u][0][e]);
          v[4 + e] = __uint_as_float(xr[u][1][e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = bf16_lo(xr[u][0][e]);
          v[2 * e + 1] = bf16_hi(xr[u][0][e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = in_activation(p.in_act, v[e], ina[e], inb[e], p.in_slope);
      const u32x4 o{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7])};
      return is_hist ? xr[u][0] : o;
    }
  };

  // Staged operands into LDS, then the weights; the new history goes out last, so the stores
  // never sit between a load and the wait for it.
  auto store_chunk = [&](int kc) __attribute__((always_inline)) {
    const bool in_range = kc * kChunk + q8 < c_in;
#pragma unroll
    for (int u = 0; u < Tile::X_PIECES; ++u) {
      const int r = (tid >> 2) + u * (NT / 4);
      const u32x4 v = stage_value(u);
      if (r < rows) *reinterpret_cast<u32x4*>(xs + r * kChunk + q8) = v;
      if constexpr (IN != IN_RAW) xr[u][0] = v;
    }
#pragma unroll
    for (int u = 0; u < Tile::W_PIECES; ++u) {
      if (wlds[u] >= 0) {
        u32x4 v;
        if constexpr (W_FP8) v = fp8x8_to_bf16x8(wr8[u]);
        else v = wr[u];
        *reinterpret_cast<u32x4*>(ws + wlds[u]) = v;
      }
    }
    if (hist != nullptr) {
#pragma unroll
      for (int u = 0; u < Tile::X_PIECES; ++u) {
        const uint32_t ho = (hwoff[u] >= 0 && in_range)
                                ? (uint32_t)(hwoff[u] + kc * kChunk) * 2 : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b128(xr[u][0], h_rsrc, ho, 0, 0);
      }
    }
  };

  f32x4 acc[TCO][TP];
#pragma unroll
  for (int c = 0; c < TCO; ++c)
#pragma unroll
    for (int t = 0; t < TP; ++t) acc[c][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lrow = lane & 15;
  const int lk = (lane >> 4) * 8;
  const int wco0 = wave_co * TCO * 16;
  const int wp0 = wave_p * TP * 16;

  // This lane's staged row for each of its position groups (tap 0).
  int xrow[TP];
#pragma unroll
  for (int t = 0; t < TP; ++t) {
    const int m = m0 + wp0 + t * 16 + lrow;
    xrow[t] = m < m_end ? (m - m0) + (m / L - b0) * halo : 0;
  }

  // The epilogue's per-column coefficients into LDS (visible after the first barrier below).
  float* coef = reinterpret_cast<float*>(
      reinterpret_cast<uint8_t*>(lds) + Tile::coef_offset(MAX_ROWS, taps, FUSE2));
  stage_coefficients<BCO, NT, FUSE2>(p, coef, n0);

  load_chunk(0);
  for (int kc = 0; kc < chunks; ++kc) {
    __syncthreads();
    store_chunk(kc);
    __syncthreads();
    if (kc + 1 < chunks) load_chunk(kc + 1);
    else if constexpr (FUSE2) load_w2();
    const u16* wtap = ws + (wco0 + lrow) * WROW + lk;
    for (int j = 0; j < taps; ++j) {
      bf16x8 a[TCO];
#pragma unroll
      for (int c = 0; c < TCO; ++c)
        a[c] = *reinterpret_cast<const bf16x8*>(wtap + c * 16 * WROW);
      const int shift = j * dil;
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const bf16x8 bv =
            *reinterpret_cast<const bf16x8*>(xs + (xrow[t] + shift) * kChunk + lk);
#pragma unroll
        for (int c = 0; c < TCO; ++c)
          acc[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c], bv, acc[c][t], 0, 0, 0);
      }
      wtap += kChunk;
    }
  }

  const int ch_in_tile = (lane >> 4) * 4;
  int coef_scale = kScale, coef_bias = kBias;

  if constexpr (FUSE2) {
    // h = mid_act(acc * scale + bias) as bf16 into LDS [BCO/32][BP][32], the four 16-byte slots
    // of a 64-byte row rotated by (row / 2) % 4 so that the operand reads of 16 rows meet no bank
    // conflict; W2 into [BCO/32][BCO][32]. (The activation is a compile-time constant of each
    // copy of the loop: one branch per tile, not one per element.)
    u16* hs = lds;
    u16* w2s = lds + BCO * BP;
    __syncthreads();
    auto put_h = [&](auto act_c) __attribute__((always_inline)) {
      constexpr int ACT = decltype(act_c)::value;
#pragma unroll
      for (int c = 0; c < TCO; ++c) {
        const int n = wco0 + c * 16 + ch_in_tile;  // n0 = 0: one column tile holds every channel
        const f32x4 sc = *reinterpret_cast<const f32x4*>(coef + kScale * BCO + n);
        const f32x4 bi = *reinterpret_cast<const f32x4*>(coef + kBias * BCO + n);
        const f32x4 ma = *reinterpret_cast<const f32x4*>(coef + kMidA * BCO + n);
        const f32x4 mb = *reinterpret_cast<const f32x4*>(coef + kMidB * BCO + n);
#pragma unroll
        for (int t = 0; t < TP; ++t) {
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            y[e] = operand_act(ACT, acc[c][t][e] * sc[e] + bi[e], ma[e], mb[e], p.mid_slope);
          uint2 o;
          o.x = pack_bf16x2(y[0], y[1]);
          o.y = pack_bf16x2(y[2], y[3]);
          const int pos = wp0 + t * 16 + lrow;
          const int slot = ((n & 31) >> 3) ^ ((pos >> 1) & 3);
          *reinterpret_cast<uint2*>(hs + ((n >> 5) * BP + pos) * kChunk + slot * 8 + (n & 7)) = o;
          acc[c][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    };
    if (p.mid_act == OMNI_ACT_SNAKE) put_h(std::integral_constant<int, OMNI_ACT_SNAKE>{});
    else if (p.mid_act == OMNI_ACT_LEAKY_RELU)
      put_h(std::integral_constant<int, OMNI_ACT_LEAKY_RELU>{});
    else put_h(std::integral_constant<int, OMNI_ACT_NONE>{});
#pragma unroll
    for (int u = 0; u < W2_PIECES; ++u) {
      const int piece = tid + u * NT;
      if (piece < BCO * BCO / 8) {
        u32x4 v;
        if constexpr (W_FP8) v = fp8x8_to_bf16x8(wr8[u]);
        else v = wr[u];
        // 64-byte rows of W2, slot s of row r holding the row's piece s ^ ((r / 2) % 4)
        *reinterpret_cast<u32x4*>(w2s + (piece ^ ((piece >> 3) & 3)) * 8) = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kc = 0; kc < BCO / kChunk; ++kc) {
      bf16x8 a[TCO];
#pragma unroll
      for (int c = 0; c < TCO; ++c)
        a[c] = *reinterpret_cast<const bf16x8*>(
            w2s + ((kc * BCO) + wco0 + c * 16 + lrow) * kChunk +
            ((((lane >> 4) ^ ((wco0 + c * 16 + lrow) >> 1)) & 3) << 3));
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const int pos = wp0 + t * 16 + lrow;
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(
            hs + (kc * BP + pos) * kChunk + (((lane >> 4) ^ ((pos >> 1) & 3)) * 8));
#pragma unroll
        for (int c = 0; c < TCO; ++c)
          acc[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c], bv, acc[c][t], 0, 0, 0);
      }
    }
    coef_scale = kScale2;
    coef_bias = kBias2;
  }

  conv_epilogue<Tile, WAVES_P, TCO, TP>(p, acc, lds, coef, coef_scale, coef_bias, n0, m0, m_end,
                                       wave_p, wco0);
}

// Raise a kernel's dynamic-LDS limit to the CU's 160 KiB. A refusal is not an error here (the
// launch check reports a launch the runtime cannot make), so its status is cleared.
inline bool raise_lds_limit(const void* kernel) {
  const hipError_t e =
      hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  (void)hipGetLastError();
  return e == hipSuccess;
}

// The kernel configuration a launcher picks from its list: by problem size (force = 0), or the
// list's force-th entry (1-based; OMNI_ERR_UNSUPPORTED when it does not fit the problem). With
// launch = false the choice is reported and nothing runs.
struct Choice {
  int force = 0;
  bool launch = true;
  int chosen = 0;           // 1-based entry of the list (out)
  int count = 0;            // entries in the list (out)
  int64_t workgroups = 0;   // of the chosen entry (out)
};

// Record the choice (the forced entry when one is asked for) and launch it unless the caller
// only asks which it would be.
template <typename RunFn>
int choose_and_launch(Choice& ch, int n, const bool* fits, const int64_t* wgs, RunFn* run,
                      int pick, const ConvParams& p, hipStream_t stream) {
  ch.count = n;
  if (ch.force > 0) {
    if (ch.force > n || !fits[ch.force - 1]) return OMNI_ERR_UNSUPPORTED;
    pick = ch.force - 1;
  }
  if (pick < 0) return OMNI_ERR_UNSUPPORTED;
  ch.chosen = pick + 1;
  ch.workgroups = wgs[pick];
  return ch.launch ? run[pick](p, stream) : OMNI_OK;
}

template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_ROWS, int MAX_TAPS>
struct Config {
  using Tile = ConvTile<WAVES_CO, WAVES_P, TCO, TP, MAX_ROWS, MAX_TAPS>;

  // Staged rows of the fullest tile: BP positions over at most nseg row segments, each with its
  // own halo.
  static int64_t rows_needed(const ConvParams& p) {
    const int64_t bp = Tile::BP;
    int64_t nseg = (bp + p.length - 2) / p.length + 1;
    if (nseg > p.batch) nseg = p.batch;
    return bp + nseg * p.halo;
  }

  static bool fits(const ConvParams& p, bool fuse2) {
    if (p.taps > MAX_TAPS || rows_needed(p) > MAX_ROWS) return false;
    if (fuse2 && p.n_cols != Tile::BCO) return false;
    return Tile::lds_bytes(MAX_ROWS, p.taps, fuse2) <= 160 * 1024;
  }

  static int64_t workgroups(const ConvParams& p) {
    const int64_t positions = (int64_t)p.batch * p.length;
    return ((positions + Tile::BP - 1) / Tile::BP) * ((p.n_cols + Tile::BCO - 1) / Tile::BCO);
  }

  template <int IN, bool W_FP8, bool FUSE2>
  static int launch_as(ConvParams p, hipStream_t stream) {
    auto k = conv_mfma_kernel<WAVES_CO, WAVES_P, TCO, TP, MAX_ROWS, MAX_TAPS, IN, W_FP8, FUSE2>;
    // The dynamic-LDS limit is raised once per kernel instantiation (to the 160 KiB maximum), on
    // its first launch, so launches inside a graph capture make no attribute calls.
    static const bool raised = raise_lds_limit((const void*)k);
    (void)raised;
    const size_t lds = Tile::lds_bytes(MAX_ROWS, p.taps, FUSE2);
    hipLaunchKernelGGL(k, dim3((unsigned)(p.p_tiles * p.n_tiles)), dim3(Tile::NT), lds, stream, p);
    OMNI_LAUNCH_CHECK();
    return OMNI_OK;
  }

  template <int IN, bool W_FP8, bool FUSE2>
  static int launch(ConvParams p, hipStream_t stream) {
    const int64_t positions = (int64_t)p.batch * p.length;
    p.p_tiles = (int)((positions + Tile::BP - 1) / Tile::BP);
    p.n_tiles = (int)((p.n_cols + Tile::BCO - 1) / Tile::BCO);
    return launch_as<IN, W_FP8, FUSE2>(p, stream);
  }
};

// Tile configurations for up to 7 taps (k <= 7 convs, k = 2s transposed convs) and up to 11 (the
// HiFiGAN k = 11 resblocks). The fused residual-unit form needs one column tile that holds every
// channel (96: 2 x 8 waves of 48 x 48; 192: 4 x 4 waves of 48 x 48; four waves per SIMD, which
// made the fp8 long form 1.10x faster than 4 / 8 waves of 96-column tiles).
template <int T>
struct Configs {
  // register budgets (accumulators + staging) keep two waves per SIMD, four for Q (16 waves,
  // tried first: fp8 long form 1.09x, HiFiGAN 1.02x faster than starting at A)
  using Q = Config<2, 8, 3, 3, 384 + 2 * kMaxHalo, T>;  // 96 x 384, 16 waves
  using A = Config<1, 4, 6, 3, 192 + 2 * kMaxHalo, T>;  // 96 cols x 192 positions, 4 waves
  using K = Config<2, 4, 6, 2, 128 + 4 * kMaxHalo, T>;  // 192 x 128, 8 waves
  using H = Config<2, 4, 4, 4, 256 + 2 * kMaxHalo, T>;  // 128 x 256, 8 waves
  using C = Config<1, 4, 4, 4, 256 + 2 * kMaxHalo, T>;  // 64 x 256
  using B = Config<2, 2, 4, 4, 128 + 3 * kMaxHalo, T>;  // 128 x 128
  using D = Config<2, 2, 4, 2, 64 + 4 * kMaxHalo, T>;   // 128 x 64
  using E = Config<2, 2, 2, 2, 64 + 4 * kMaxHalo, T>;   // 64 x 64
  using F = Config<4, 1, 2, 2, 32 + 4 * kMaxHalo, T>;   // 128 x 32
  using S = Config<1, 8, 2, 4, 512 + 2 * kMaxHalo, T>;  // 32 x 512, 8 waves (32-channel layers)
  static constexpr int kCount = 10;

  // The list in order of measured efficiency on MI355X (entry k of a forced choice is the k-th):
  // the first configuration that fits, wastes at most an eighth of its column tiles and still
  // gives at least half a workgroup per CU; failing that (small problems), the fitting one with
  // the most workgroups. The 32-column tile comes last: it is for layers with 32 output columns,
  // where every wider tile wastes most of its matrix work.
  template <int IN, bool W_FP8>
  static int launch(const ConvParams& p, Choice& ch, hipStream_t stream) {
    constexpr int64_t min_wgs = 128;
    const bool fits[kCount] = {Q::fits(p, false), A::fits(p, false), K::fits(p, false),
                               H::fits(p, false), C::fits(p, false), B::fits(p, false),
                               D::fits(p, false), E::fits(p, false), F::fits(p, false),
                               S::fits(p, false)};
    const int64_t wgs[kCount] = {Q::workgroups(p), A::workgroups(p), K::workgroups(p),
                                 H::workgroups(p), C::workgroups(p), B::workgroups(p),
                                 D::workgroups(p), E::workgroups(p), F::workgroups(p),
                                 S::workgroups(p)};
    const int bco[kCount] = {Q::Tile::BCO, A::Tile::BCO, K::Tile::BCO, H::Tile::BCO,
                             C::Tile::BCO, B::Tile::BCO, D::Tile::BCO, E::Tile::BCO,
                             F::Tile::BCO, S::Tile::BCO};
    int (*const run[kCount])(ConvParams, hipStream_t) = {
        &Q::template launch<IN, W_FP8, false>, &A::template launch<IN, W_FP8, false>,
        &K::template launch<IN, W_FP8, false>, &H::template launch<IN, W_FP8, false>,
        &C::template launch<IN, W_FP8, false>, &B::template launch<IN, W_FP8, false>,
        &D::template launch<IN, W_FP8, false>, &E::template launch<IN, W_FP8, false>,
        &F::template launch<IN, W_FP8, false>, &S::template launch<IN, W_FP8, false>};
    int pick = -1, most = -1;
    for (int i = 0; i < kCount; ++i) {
      if (!fits[i]) continue;
      const int64_t padded = (p.n_cols + bco[i] - 1) / bco[i] * bco[i];
      if (pick < 0 && wgs[i] >= min_wgs && (padded - p.n_cols) * 8 <= p.n_cols) pick = i;
      if (most < 0 || wgs[i] > wgs[most]) most = i;
    }
    if (pick < 0) pick = most;
    return choose_and_launch(ch, kCount, fits, wgs, run, pick, p, stream);
  }
};

using ResidualUnit96 = Config<2, 8, 3, 3, 384 + 2 * kMaxHalo, 7>;       // fused, 96 channels
using ResidualUnit96Short = Config<1, 2, 6, 1, 32 + 4 * kMaxHalo, 7>;   // short rows
using ResidualUnit192 = Config<4, 4, 3, 3, 192 + 3 * kMaxHalo, 7>;      // fused, 192 channels
using ResidualUnit192Short = Config<2, 2, 6, 1, 32 + 4 * kMaxHalo, 7>;  // short rows

// Launchers, one translation unit each (they compile in parallel): taps <= 7 for each input and
// weight dtype, taps <= 11 for bf16 weights, and the fused residual-unit forms.
template <int IN, bool W_FP8>
int launch_taps7(const ConvParams& p, Choice& ch, hipStream_t stream);
int launch_taps11(const ConvParams& p, int in_mode, Choice& ch, hipStream_t stream);
template <bool W_FP8>
int launch_fused(const ConvParams& p, int in_mode, Choice& ch, hipStream_t stream);
#define OMNI_DECLARE_TAPS7(IN_, FP8_) \
  template <> int launch_taps7<IN_, FP8_>(const ConvParams& p, Choice& ch, hipStream_t stream);
OMNI_DECLARE_TAPS7(IN_RAW, false)
OMNI_DECLARE_TAPS7(IN_RAW, true)
OMNI_DECLARE_TAPS7(IN_ACT, false)
OMNI_DECLARE_TAPS7(IN_ACT, true)
OMNI_DECLARE_TAPS7(IN_F32, false)
OMNI_DECLARE_TAPS7(IN_F32, true)
#undef OMNI_DECLARE_TAPS7
template <> int launch_fused<false>(const ConvParams& p, int in_mode, Choice& ch, hipStream_t stream);
template <> int launch_fused<true>(const ConvParams& p, int in_mode, Choice& ch, hipStream_t stream);

}  // namespace omni_conv
