// The residual units of a decoder block in one kernel (gfx950 bf16 MFMA).
//
// A DAC decoder block ends in residual units u -> conv k7 (dilation 1, 3, 9) -> Snake -> conv k1
// -> + x. Run one launch per unit, the float32 residual stream x and the bf16 operand travel
// through HBM between every unit (12 bytes per element per unit at the 96-channel stage). Here a
// workgroup owns a tile of positions and runs every unit over it with x held in registers:
//
//   * staged rows: each row segment of the tile is preceded by H = sum of the unit halos rows
//     (the causal receptive field of the whole stack), so the last unit's outputs for the tile's
//     positions depend only on staged data. Unit k computes every staged row; a row whose window
//     reaches before the segment's first staged row gives a value no later unit's valid row
//     reads (row q of a segment is exact for unit k once q >= halo_1 + ... + halo_k).
//   * x: float32 in the MFMA accumulator layout (lane = row, 4 consecutive channels per lane),
//     loaded once from HBM (float32, or a float16 residual stream widened exactly), updated in
//     place by each unit's k = 1 conv.
//   * the operand u_k = Snake(x_k) and the h tile between the two convs: bf16 in one LDS tile
//     [C/32][guard + rows][32] (64-byte rows, 16-byte slot s of row r stored at s ^ ((r / 2) % 4),
//     so an operand read of 16 consecutive rows from any first row meets no bank conflict);
//     guard rows ahead of row 0 keep the taps of the first rows inside the tile.
//   * weights: by LDS DMA into a two-buffer ring of stages (a 32-channel chunk of the dilated
//     conv, or the k = 1 conv), the next stage's DMA running during this stage's MFMAs; bf16
//     weights as they are (a column's taps in a 256-byte row, 16-byte slot s of column n at
//     s ^ (n % 16); the k = 1 conv's 64-byte rows swizzled as the operand tile's, so the weight
//     reads meet no bank conflict either), E4M3 weights as bytes widened to bf16 (exactly) when
//     read.
//   * long rows (sweep): a workgroup runs consecutive tiles of one stream row, and each operand's
//     last halo rows pass from one tile to the next through LDS instead of being recomputed.
//   * streaming: rows left of position 0 of a stream row take each unit's own history copy (or
//     zeros), and the workgroup that owns the last 6 * d positions of a row writes them as the
//     unit's new history, as the one-unit kernel does.
//
// Only the last unit's operand-to-be, Snake(x_last), leaves as bf16 (and x_last as float32 on
// request). The arithmetic of every element repeats the one-unit kernel's expression for
// expression, so the two paths give the same bits.
#pragma once

#include "conv_kernel.h"

namespace omni_stack {

using omni_conv::fp8x8_to_bf16x8;
using omni_conv::kChunk;
using omni_conv::pack_bf16x2;

constexpr int kMaxUnits = OMNI_MAX_RESIDUAL_UNITS;
constexpr int kTaps = 7;    // the residual unit's dilated conv
constexpr int kGuard = 64;  // LDS rows ahead of row 0: the largest unit halo taken (6 * 10 = 60)
// The sweep form (a workgroup runs consecutive tiles of one stream row): the largest unit or
// final-conv halo it takes (6 * 9 = 54), the units its coefficient table holds, and the rows of
// its halo store (the dilations 1, 3, 9 and a final conv of up to 7 taps: 6 + 18 + 54 + 6)
constexpr int kSweepGuard = 56;
constexpr int kSweepUnits = 3;
constexpr int kSweepHaloRows = 84;
constexpr int kCoefRows = 8;

struct StackUnit {
  const void* w1;  // [C/32][C][7][32]
  const float* w1_scale;
  const float* b1;
  const float* in_a;  // Snake of the unit's input
  const float* in_b;
  const float* mid_a;  // Snake between the two convs
  const float* mid_b;
  const void* w2;  // [C/32][C][32]
  const float* w2_scale;
  const float* b2;
  u16* hist;  // history pool of the dilated conv's operand, or NULL
  int hist_stride;
  int dil, halo;
  uint32_t w1_bytes, w2_bytes, hist_bytes;
};

struct StackParams {
  const void* x;  // float32, or float16 when x_f16 (x_out likewise)
  int x_f16;
  int x_sb, x_st;
  int batch, length;
  int nunits;
  StackUnit unit[kMaxUnits];
  const int64_t* slot_index;
  const int64_t* slot_parity;
  int64_t hist_slots;
  int hist_cold;
  const float* out_a;
  const float* out_b;
  u16* out;
  int o_sb, o_st;
  void* x_out;
  int xo_sb, xo_st;
  uint32_t x_bytes, o_bytes, xo_bytes;
  // the decoder's final conv to one channel (fin_w != NULL): [fin_taps][C] float32 weights
  const float* fin_w;
  const float* fin_b;
  int fin_taps, fin_act;
  u16* fin_hist;  // [slots][2][fin_taps - 1][C] bf16, or NULL
  int fin_hist_stride;
  uint32_t fin_hist_bytes;
  float* fin_out;
  int64_t fin_o_sb;
  const float* coef_table;  // the coefficient rows below, precomputed (stack_coef), or NULL
  int H;              // staged rows ahead of each segment (sum of the unit halos and the
                      // final conv's taps - 1)
  int seg_len;        // long rows: output positions per tile; short rows: the row length
  int tiles_per_row;  // long rows: tiles per stream row; 0: short rows, whole rows per tile
  int rows_per_tile;  // short rows: stream rows per tile
  int sweep_segments;   // sweep: workgroups per stream row
  int sweep_positions;  // sweep: positions per workgroup (the last one of a row may hold fewer)
  // sweep: the halo store's rows of operand k (unit k's input; k = nunits: the final conv's)
  // and where they start
  int halo_rows[kMaxUnits + 1];
  int halo_off[kMaxUnits + 1];
};

// LDS element offset of 16-byte slot `slot` of staged row `row` (guard included) in chunk kc.
template <int UROWS>
__device__ __forceinline__ int uaddr(int kc, int row, int slot) {
  return (kc * UROWS + row) * kChunk + ((slot ^ ((row >> 1) & 3)) << 3);
}

// The per-launch coefficient rows in LDS order: per unit kCoefRows rows of C (scale1, bias1,
// mid Snake a in revolutions, b, scale2, bias2, the next operand's Snake a in revolutions, b),
// then unit 0's input Snake (a in revolutions, b). Entry e of the table.
enum { kS1, kB1, kMA, kMB, kS2, kB2, kNA, kNB };

__device__ __forceinline__ float stack_coef(const StackParams& p, int e, int C) {
  const int k = e / C;
  const int n = e - k * C;
  if (k >= p.nunits * kCoefRows)
    return k == p.nunits * kCoefRows ? p.unit[0].in_a[n] * kInvTwoPi : p.unit[0].in_b[n];
  const int unit = k / kCoefRows;
  const int row = k - unit * kCoefRows;
  const StackUnit& U = p.unit[unit];
  const bool last = unit + 1 == p.nunits;
  switch (row) {
    case kS1: return U.w1_scale ? U.w1_scale[n] : 1.f;
    case kB1: return U.b1 ? U.b1[n] : 0.f;
    case kMA: return U.mid_a[n] * kInvTwoPi;
    case kMB: return U.mid_b[n];
    case kS2: return U.w2_scale ? U.w2_scale[n] : 1.f;
    case kB2: return U.b2 ? U.b2[n] : 0.f;
    case kNA: return (last ? p.out_a[n] : p.unit[unit + 1].in_a[n]) * kInvTwoPi;
    default: return last ? p.out_b[n] : p.unit[unit + 1].in_b[n];
  }
}

template <int C>
__global__ void stack_coef_kernel(const StackParams p, float* table) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < (p.nunits * kCoefRows + 2) * C) table[e] = stack_coef(p, e, C);
}

template <int C, int WCO, int WP, int TP, bool SWEEP = false, bool W8 = false>
struct StackTile {
  static constexpr int NT = 64 * WCO * WP;
  static constexpr int TCO = C / (16 * WCO);
  static constexpr int R = WP * TP * 16;  // staged rows per tile
  static constexpr int CH = C / kChunk;
  // LDS rows ahead of row 0, holding the halo rows a unit's dilated conv reads before the tile's
  // first row (zeros, or in the sweep the previous tile's last rows of the unit's operand)
  static constexpr int GUARD = SWEEP ? kSweepGuard : kGuard;
  static constexpr int UROWS = GUARD + R;
  // LDS DMA ring: two buffers, each holding one stage of weights as they are stored (bf16, or
  // E4M3 bytes widened when read): the dilated conv's chunk kc for taps 0-3 or 4-6 (bf16: [C]
  // rows of 16 slots, slot s of row n at s ^ (n % 16), taps 4-6 using 12 of them) or all 7 taps
  // (E4M3: [C][7 * 32 bytes + one 16-byte pad], an odd multiple of 16 bytes), or the k = 1 conv
  // ([C/32][C][32]; bf16 rows swizzled as the operand tile's); a stage is whole 64-lane DMA
  // instructions of 16 bytes.
  static constexpr int WE = W8 ? 1 : 2;              // bytes per weight
  static constexpr int P_LO = W8 ? 7 * 2 + 1 : 16;   // 16-byte slots per weight row, taps 0-6
                                                     // (E4M3, +1 pad) or 0-3 (bf16)
  static constexpr int P_HI = 16;                    // bf16 taps 4-6
  static constexpr int RING_SLOTS = (C * P_LO + 63) / 64 * 64;
  static constexpr int RING_ELEMS = RING_SLOTS * 8;
  static constexpr int W2_SLOTS = CH * C * 2 * WE;   // the k = 1 conv's weights
  static constexpr int CONV_STAGES = W8 ? CH : 2 * CH;  // per unit: chunks (x 2 tap halves)
  static constexpr int STAGES = CONV_STAGES + 1;        // then the k = 1 conv
  static_assert(W2_SLOTS <= RING_SLOTS, "the k = 1 weights fit one ring buffer");
  static constexpr int W_ELEMS = 2 * RING_ELEMS;
  static constexpr int UNITS = SWEEP ? kSweepUnits : kMaxUnits;  // units the coefficients hold
  static constexpr int COEF = (UNITS * kCoefRows + 2) * C;  // floats
  // the sweep's halo store: per unit input operand and the final conv's, the previous tile's
  // last rows ([HALO_ROWS][C] bf16, rows of the operands in order)
  static constexpr int HALO_ROWS = SWEEP ? kSweepHaloRows : 0;
  static constexpr size_t lds_bytes() {
    return (size_t)CH * UROWS * kChunk * 2 + (size_t)W_ELEMS * 2 + (size_t)COEF * 4 +
           (size_t)HALO_ROWS * C * 2;
  }
  static_assert(C % (16 * WCO) == 0 && C % kChunk == 0, "tile shape");
  static_assert(R % 16 == 0, "staged rows in 16-row groups");
};

template <int C, int WCO, int WP, int TP, bool W_FP8, bool SWEEP>
__global__ void __launch_bounds__(64 * WCO * WP) residual_stack_kernel(const StackParams p) {
  using Tile = StackTile<C, WCO, WP, TP, SWEEP, W_FP8>;
  constexpr int GUARD = Tile::GUARD;
  constexpr int NT = Tile::NT;
  constexpr int TCO = Tile::TCO;
  constexpr int CH = Tile::CH;
  constexpr int UROWS = Tile::UROWS;
  constexpr int PIECES_PER_ROW = C / 8;  // 16-byte pieces of a staged row
  extern __shared__ __attribute__((aligned(16))) u16 lds[];
  u16* us = lds;                        // operand / h tile
  u16* ws = lds + CH * UROWS * kChunk;  // weights
  float* coef = reinterpret_cast<float*>(ws + Tile::W_ELEMS);
  float* in0 = coef + p.nunits * kCoefRows * C;  // unit 0's input Snake a, b
  u16* halo = reinterpret_cast<u16*>(coef + Tile::COEF);  // the sweep's halo store

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wave_co = wave % WCO;
  const int wave_p = wave / WCO;
  const int lrow = lane & 15;
  const int lk = (lane >> 4) * 8;
  const int wco0 = wave_co * TCO * 16;
  const uint32_t xsize = p.x_f16 ? 2u : 4u;  // bytes per element of x and x_out

  // The workgroup's positions: nseg row segments of len positions from position i0 of rows b0..
  // (one tile), or in the sweep the positions [i0, seg_end) of row b0, tile after tile.
  int b0, i0, nseg, len, seg_end = 0;
  if constexpr (SWEEP) {
    b0 = blockIdx.x / p.sweep_segments;
    i0 = (blockIdx.x - b0 * p.sweep_segments) * p.sweep_positions;
    seg_end = min(p.length, i0 + p.sweep_positions);
    nseg = 1;
    len = 0;  // set per tile
  } else if (p.tiles_per_row > 0) {
    b0 = blockIdx.x / p.tiles_per_row;
    i0 = (blockIdx.x - b0 * p.tiles_per_row) * p.seg_len;
    nseg = 1;
    len = min(p.seg_len, p.length - i0);
  } else {
    b0 = blockIdx.x * p.rows_per_tile;
    i0 = 0;
    nseg = min(p.rows_per_tile, p.batch - b0);
    len = p.length;
  }
  const int L = p.length;
  // The final conv's weights ([fin_taps][C] float32, at most 8 taps), rounded to bf16 once per
  // workgroup and held in registers as this lane's A operand of its taps-as-columns MFMA: tap
  // lane % 16 (zeros past the taps), channels 8 (lane / 16) .. + 7 of each 32-channel chunk.
  static_assert(kTaps + 1 <= 16, "a tap per A-operand row");
  bf16x8 fin_a[CH];
#pragma unroll
  for (int kc = 0; kc < CH; ++kc) fin_a[kc] = bf16x8{};
  if (p.fin_w != nullptr && (lane & 15) < p.fin_taps) {
    const float* wrow = p.fin_w + (lane & 15) * C + (lane >> 4) * 8;
#pragma unroll
    for (int kc = 0; kc < CH; ++kc) {
      const float* wk = wrow + kc * kChunk;
      fin_a[kc] = __builtin_bit_cast(
          bf16x8, u32x4{pack_bf16x2(wk[0], wk[1]), pack_bf16x2(wk[2], wk[3]),
                        pack_bf16x2(wk[4], wk[5]), pack_bf16x2(wk[6], wk[7])});
    }
  }
  // ---- set-up, once per workgroup: coefficients, zero guard rows (and halo store) in LDS
  const int ncoef = (p.nunits * kCoefRows + 2) * C;
  if (p.coef_table != nullptr) {
    // a straight copy of the precomputed rows: independent 16-byte loads
    for (int e = tid * 4; e < ncoef; e += NT * 4)
      *reinterpret_cast<f32x4*>(coef + e) = *reinterpret_cast<const f32x4*>(p.coef_table + e);
  } else {
    for (int e = tid; e < ncoef; e += NT) coef[e] = stack_coef(p, e, C);
  }
  for (int e = tid; e < CH * GUARD * 4; e += NT) {
    const int kc = e / (GUARD * 4);
    const int rem = e - kc * GUARD * 4;
    *reinterpret_cast<u32x4*>(us + (kc * UROWS + (rem >> 2)) * kChunk + (rem & 3) * 8) =
        u32x4{0u, 0u, 0u, 0u};
  }
  if constexpr (SWEEP) {
    for (int e = tid; e < Tile::HALO_ROWS * C / 8; e += NT)
      *reinterpret_cast<u32x4*>(halo + e * 8) = u32x4{0u, 0u, 0u, 0u};
  }

  // DMA of weight stage g (g = unit * STAGES + r: r < CONV_STAGES the dilated conv's chunk, with
  // bf16 weights r / 2 for taps 0-3 or 4-6, with E4M3 weights r for all taps; r = CONV_STAGES
  // the k = 1 conv) into ring buffer g % 2: this wave's share of the stage's 64-lane 16-byte
  // instructions. Lane i of an instruction fills ring slot 64 * instr + i, so each lane loads the
  // global piece that belongs in its slot (pad slots reload the chunk's first piece).
  //
  // The per-lane byte offsets of the dilated-conv patterns (bf16 taps 0-3: 17 slots per column
  // row, taps 4-6: 13; E4M3 taps 0-6: 15) are the same for every chunk and unit up to the chunk's
  // base, which goes in the scalar offset, so they are computed once here.
  constexpr int NWAVES = NT / 64;
  constexpr int LO_INSTRS = (C * Tile::P_LO + 63) / 64;
  constexpr int HI_INSTRS = W_FP8 ? 0 : (C * Tile::P_HI + 63) / 64;
  constexpr int W2_INSTRS = Tile::W2_SLOTS / 64;
  static_assert(Tile::W2_SLOTS % 64 == 0, "the k = 1 stage is whole DMA instructions");
  constexpr int LO_PER_WAVE = (LO_INSTRS + NWAVES - 1) / NWAVES;
  constexpr int HI_PER_WAVE = (HI_INSTRS + NWAVES - 1) / NWAVES;
  uint32_t lo_off[LO_PER_WAVE], hi_off[HI_PER_WAVE > 0 ? HI_PER_WAVE : 1];
  {
    // slot j of column row n holds bytes s * 16 .. of the column's taps t0 .. t0 + nt - 1
    // (packed [C][7][32] per chunk), s = j (E4M3) or j ^ (n % 16) (bf16)
    auto slot_offset = [&](int di, int P, int t0, int nt) __attribute__((always_inline)) {
      const int slot = di * 64 + lane;
      const int n = slot / P;
      const int j = slot - n * P;
      const int s = W_FP8 ? j : j ^ (n & 15);
      return (n < C && s < nt * 2 * Tile::WE)
                 ? (uint32_t)((n * kTaps + t0) * kChunk * Tile::WE + s * 16) : 0u;
    };
#pragma unroll
    for (int i = 0; i < LO_PER_WAVE; ++i)
      lo_off[i] = slot_offset(wave + i * NWAVES, Tile::P_LO, 0, W_FP8 ? kTaps : 4);
#pragma unroll
    for (int i = 0; i < HI_PER_WAVE; ++i) hi_off[i] = slot_offset(wave + i * NWAVES, Tile::P_HI, 4, 3);
  }
  auto dma_stage = [&](int g) __attribute__((always_inline)) {
    {
      const int k = g / Tile::STAGES;
      const int r = g - k * Tile::STAGES;
      if (k >= p.nunits) return;
      u16* buf = ws + (g & 1) * Tile::RING_ELEMS;
      if (r < Tile::CONV_STAGES) {
        const auto rs = buffer_rsrc(p.unit[k].w1, p.unit[k].w1_bytes);
        const int chunk = W_FP8 ? r : r >> 1;
        const int chunk_base = chunk * C * kTaps * kChunk * Tile::WE;  // bytes
        if (!W_FP8 && (r & 1)) {
#pragma unroll
          for (int i = 0; i < HI_PER_WAVE; ++i) {
            const int di = wave + i * NWAVES;
            if (di < HI_INSTRS)
              __builtin_amdgcn_raw_ptr_buffer_load_lds(
                  rs, (__attribute__((address_space(3))) void*)(buf + di * 64 * 8), 16,
                  (int)hi_off[i], chunk_base, 0, 0);
          }
        } else {
#pragma unroll
          for (int i = 0; i < LO_PER_WAVE; ++i) {
            const int di = wave + i * NWAVES;
            if (di < LO_INSTRS)
              __builtin_amdgcn_raw_ptr_buffer_load_lds(
                  rs, (__attribute__((address_space(3))) void*)(buf + di * 64 * 8), 16,
                  (int)lo_off[i], chunk_base, 0, 0);
          }
        }
      } else {
        const auto rs = buffer_rsrc(p.unit[k].w2, p.unit[k].w2_bytes);
#pragma unroll
        for (int i = 0; i < (W2_INSTRS + NWAVES - 1) / NWAVES; ++i) {
          const int di = wave + i * NWAVES;
          // bf16: slot s of 64-byte row r (four slots) holds piece s ^ ((r / 2) % 4) of the row
          const int slot = di * 64 + lane;
          const int src = W_FP8 ? slot : (slot ^ ((slot >> 3) & 3));
          if (di < W2_INSTRS)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)(buf + di * 64 * 8), 16,
                (int)((uint32_t)src * 16u), 0, 0, 0);
        }
      }
    }
  };
  // Start of weight stage g: this wave's DMA of stage g is complete, then every wave's (the
  // barrier), which also retires every read of the other buffer; stage g + 1 goes into it.
  auto stage_begin = [&](int g) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    dma_stage(g + 1);
  };

  // LDS addressing of the operand tile from the accumulator layout. Staged rows of this lane are
  // row0 + 16 t, so the slot swizzle (row / 2) % 4 is row0's for every t: each access is a
  // per-lane base plus a compile-time offset.
  const int row0 = GUARD + wave_p * TP * 16 + lrow;  // staged row of t = 0 (guard included)
  const int sw = (row0 >> 1) & 3;
  // columns n = c * 16 + (lane / 16) * 4 .. + 3 of the lane: chunk c / 2, 16-byte slot
  // 2 * (c % 2) + lane / 32, element (lane / 16 % 2) * 4 within the slot
  const int put_base0 = row0 * kChunk + ((((lane >> 5)) ^ sw) << 3) + ((lane >> 4) & 1) * 4;
  const int put_base1 = row0 * kChunk + (((2 | (lane >> 5)) ^ sw) << 3) + ((lane >> 4) & 1) * 4;
  const int rd_base = row0 * kChunk + (((lane >> 4) ^ sw) << 3);  // operand reads at row0 + 16t
  static_assert(WCO == 1, "the column layout below assumes one wave holds every column");
  auto put = [&](int c, int t, float y0, float y1, float y2, float y3) __attribute__((always_inline)) {
    uint2 o;
    o.x = pack_bf16x2(y0, y1);
    o.y = pack_bf16x2(y2, y3);
    const int base = (c & 1) ? put_base1 : put_base0;
    *reinterpret_cast<uint2*>(us + base + (c >> 1) * UROWS * kChunk + t * 16 * kChunk) = o;
  };

  // ---- the tiles: one (nseg row segments), or in the sweep consecutive tiles of one row, the
  // first staging the causal halo H of the whole stack ahead of its positions, the later ones
  // taking each operand's halo from the previous tile (the halo store, copied into the guard)
  f32x4 xv[TCO][TP];
  f32x4 acc[TCO][TP];
  bool x_ready = false;  // xv already holds this tile's x (loaded during the previous tile)
  for (int tile = 0;; ++tile) {
  const int H = (SWEEP && tile > 0) ? 0 : p.H;
  if constexpr (SWEEP) len = min(Tile::R - H, seg_end - i0);
  const bool has_next = SWEEP && i0 + len < seg_end;  // then this tile holds R rows
  const int span = len + H;  // staged rows per segment
  const int rows = nseg * span;

  // This lane's staged row t in the accumulator layout, its segment, stream row and position
  // (recomputed where needed rather than held in registers; in the sweep every row is of row b0)
  // (lr: the lane's row within its 16-row groups, lane % 16)
  auto row_of = [&](int t, int lr) __attribute__((always_inline)) -> int {
    return wave_p * TP * 16 + t * 16 + lr;
  };
  auto seg_of = [&](int t, int lr) __attribute__((always_inline)) -> int {
    return SWEEP ? 0 : row_of(t, lr) / span;
  };
  auto pos_of = [&](int t, int lr) __attribute__((always_inline)) -> int {
    const int r = row_of(t, lr);
    return r < rows ? i0 - H + (r - seg_of(t, lr) * span) : -(1 << 30);
  };
  if (tile > 0) __syncthreads();  // the previous tile's reads of the tile, guard and ring are done
  // A wave none of whose rows is staged (the short last tile of a sweep) skips the matrix and
  // element work of every unit: no staged row reads a later row, so nothing reads its rows. It
  // still issues its share of each weight stage's DMA, meets every barrier and moves its halo
  // rows (the guard rows the first wave reads), and its SIMD's other wave runs alone.
  const bool active = wave_p * TP * 16 < rows;
  if (!x_ready) {
    const auto xr = buffer_rsrc(p.x, p.x_bytes);
    const int ln = opaque_copy(lane);
#pragma unroll
    for (int c = 0; c < TCO; ++c) {
      const int n = wco0 + c * 16 + (ln >> 4) * 4;
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const int pos = pos_of(t, ln & 15);
        const bool ok = pos >= 0 && pos < L;
        const uint32_t off =
            ok ? (uint32_t)((b0 + seg_of(t, ln & 15)) * p.x_sb + pos * p.x_st + n) * xsize
               : kOutOfRange;
        // raw bits (widened at unit 0's operand, where the load is first waited for)
        xv[c][t] = __builtin_bit_cast(f32x4, omni_conv::load_residual4_raw(xr, off, p.x_f16));
      }
    }
  }
  // The sweep's halo rows of operand k, once the wave has written its rows of the operand: for
  // each of the operand's last halo rows that this wave owns, move the halo store's old row (the
  // previous tile's, zeros in the first tile) into the guard row the operand's conv reads before
  // row 0 (the guard row r - R sits R rows before row r), then, when another tile follows, keep
  // the new row there. Only this wave reads and writes these rows of the store, and its LDS
  // operations complete in order, so no barrier is needed; the guard is free (every wave has
  // passed the barrier that ends the previous reader of the guard).
  auto halo_move = [&](int k) __attribute__((always_inline)) {
    if constexpr (SWEEP) {
      const int first = Tile::R - p.halo_rows[k];
      const int w0 = wave_p * TP * 16;
      const int lo = first > w0 ? first : w0;
      const int n = (w0 + TP * 16 - lo) * PIECES_PER_ROW;
      for (int e = opaque_copy(lane); e < n; e += 64) {
        const int r = lo + e / PIECES_PER_ROW;
        const int piece = e - (r - lo) * PIECES_PER_ROW;
        u32x4* st = reinterpret_cast<u32x4*>(halo + (p.halo_off[k] + r - first) * C + piece * 8);
        const u32x4 old = *st;
        const u32x4 cur =
            *reinterpret_cast<const u32x4*>(us + uaddr<UROWS>(piece >> 2, GUARD + r, piece & 3));
        *reinterpret_cast<u32x4*>(us + uaddr<UROWS>(piece >> 2, GUARD + r - Tile::R, piece & 3)) =
            old;
        if (has_next) *st = cur;
      }
    }
  };

  dma_stage(0);
  if (tile == 0) __syncthreads();  // coefficients and guard rows
  // unit 0's operand
#pragma unroll
  for (int c = 0; c < TCO; ++c) {
    if (!active) break;
    const int n = wco0 + c * 16 + (lane >> 4) * 4;
    const f32x4 a = *reinterpret_cast<const f32x4*>(in0 + n);
    const f32x4 b = *reinterpret_cast<const f32x4*>(in0 + C + n);
#pragma unroll
    for (int t = 0; t < TP; ++t) {
      const f32x4 v = omni_conv::widen_residual4(__builtin_bit_cast(u32x4, xv[c][t]), p.x_f16);
      xv[c][t] = v;
      put(c, t, snake_rev(v[0], a[0], b[0]), snake_rev(v[1], a[1], b[1]),
          snake_rev(v[2], a[2], b[2]), snake_rev(v[3], a[3], b[3]));
    }
  }
  halo_move(0);

  for (int k = 0; k < p.nunits; ++k) {
    const int h = p.unit[k].halo;
    const int d = p.unit[k].dil;
    u16* hist = p.unit[k].hist;
    const auto hr = buffer_rsrc(hist, p.unit[k].hist_bytes);
    const int hstride = p.unit[k].hist_stride;
    // the operand tile is complete (every wave's (f) of the previous unit): the unit's first
    // weight stage's barrier is that point; (a) and (b) below touch only rows that the dilated
    // conv reads after it
    stage_begin(k * Tile::STAGES);
    // (a) operand rows left of position 0 (segments that start a stream row): the history copy
    // of the row's slot, or zeros
    if (i0 == 0 && h > 0) {
      for (int e = opaque_copy(tid); e < nseg * h * PIECES_PER_ROW; e += NT) {
        const int s = e / (h * PIECES_PER_ROW);
        const int rem = e - s * h * PIECES_PER_ROW;
        const int j = rem / PIECES_PER_ROW;  // sample j of the history: position j - h
        const int piece = rem - j * PIECES_PER_ROW;
        uint32_t off = kOutOfRange;
        if (hist != nullptr && !p.hist_cold) {
          const int64_t slot = p.slot_index[b0 + s];
          if (slot >= 0 && slot < p.hist_slots) {
            const int parity = (int)(p.slot_parity[slot] & 1);
            off = (uint32_t)((int)slot * hstride + (parity * h + j) * C + piece * 8) * 2;
          }
        }
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(hr, off, 0, 0);
        const int row = GUARD + s * span + H - h + j;
        *reinterpret_cast<u32x4*>(us + uaddr<UROWS>(piece >> 2, row, piece & 3)) = v;
      }
      __syncthreads();
    }
    // (b) the new history: the last h operand samples of each stream row, written by the
    // workgroup holding them (those left of 0 by the one holding position 0); a tile that holds
    // neither a row's last h positions nor its start skips the loop (and its slot loads)
    if (hist != nullptr && (i0 == 0 || i0 + len > L - h)) {
      for (int e = opaque_copy(tid); e < nseg * h * PIECES_PER_ROW; e += NT) {
        const int s = e / (h * PIECES_PER_ROW);
        const int rem = e - s * h * PIECES_PER_ROW;
        const int j = rem / PIECES_PER_ROW;
        const int piece = rem - j * PIECES_PER_ROW;
        const int pos = L - h + j;
        const bool own = pos >= 0 ? (pos >= i0 && pos < i0 + len) : i0 == 0;
        const int64_t slot = p.slot_index[b0 + s];
        if (own && slot >= 0 && slot < p.hist_slots) {
          const int parity = (int)(p.slot_parity[slot] & 1);
          const int row = GUARD + s * span + (pos - i0) + H;
          const u32x4 v = *reinterpret_cast<const u32x4*>(us + uaddr<UROWS>(piece >> 2, row, piece & 3));
          const uint32_t off = (uint32_t)((int)slot * hstride + ((1 - parity) * h + j) * C + piece * 8) * 2;
          __builtin_amdgcn_raw_buffer_store_b128(v, hr, off, 0, 0);
        }
      }
    }
    // (c) the dilated conv
#pragma unroll
    for (int c = 0; c < TCO; ++c)
#pragma unroll
      for (int t = 0; t < TP; ++t) acc[c][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    {
      // One weight stage of NTAPS taps (E4M3 weights), software-pipelined in a fixed issue order. The stage's
      // weight tiles (tap-major, then column tile) pass through a ring of three registers: tile
      // i + 3 is read as soon as tile i's TP MFMAs have issued, two column tiles ahead of its
      // use; the next tap's TP operand tiles go to the second of two buffers while the current
      // tap's MFMAs run. So only the stage's first reads wait on LDS latency, with no more
      // operand registers than a tap's tiles (scheduling barriers keep the compiler from
      // regrouping the reads). E4M3 weights stay as loaded bytes until their MFMAs. The MFMAs
      // of each accumulator keep the order of the taps, so the sums are those of the plain loop.
      auto conv_stage = [&](auto ntaps, const u16* wtap, const u16* ukc, int t0)
          __attribute__((always_inline)) {
        constexpr int NTAPS = decltype(ntaps)::value;
        constexpr int NTILES = NTAPS * TCO;
        // u16 elements per weight row of the stage
        constexpr int P8 = Tile::P_LO * 8;
        using WRaw = typename std::conditional<W_FP8, u32x2, bf16x8>::type;
        auto load_a = [&](int i) __attribute__((always_inline)) -> WRaw {
          const int jj = i / TCO;
          const int c = i - jj * TCO;
          return *reinterpret_cast<const WRaw*>(wtap + jj * (kChunk * Tile::WE / 2) + c * 16 * P8);
        };
        auto widen = [&](const WRaw& w) __attribute__((always_inline)) -> bf16x8 {
          if constexpr (W_FP8)
            return __builtin_bit_cast(bf16x8, fp8x8_to_bf16x8(w));
          else
            return w;
        };
        auto load_b = [&](int jj, bf16x8 (&b)[TP]) __attribute__((always_inline)) {
          const int rj = row0 + (t0 + jj) * d - h;
          const int bj = rj * kChunk + (((lane >> 4) ^ ((rj >> 1) & 3)) << 3);
#pragma unroll
          for (int t = 0; t < TP; ++t)
            b[t] = *reinterpret_cast<const bf16x8*>(ukc + bj + t * 16 * kChunk);
        };
        WRaw ring[3];
        bf16x8 bb[2][TP];
        load_b(0, bb[0]);
#pragma unroll
        for (int i = 0; i < 3; ++i) ring[i] = load_a(i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jj = 0; jj < NTAPS; ++jj) {
#pragma unroll
          for (int c = 0; c < TCO; ++c) {
            const int i = jj * TCO + c;
            const bf16x8 av = widen(ring[i % 3]);
#pragma unroll
            for (int t = 0; t < TP; ++t)
              acc[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bb[jj & 1][t], acc[c][t], 0, 0, 0);
            if (i + 3 < NTILES) ring[i % 3] = load_a(i + 3);
            if (c == 1 && jj + 1 < NTAPS) load_b(jj + 1, bb[(jj + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      };
      for (int r = 0; r < Tile::CONV_STAGES; ++r) {
        const int g = k * Tile::STAGES + r;
        if (r > 0) stage_begin(g);  // stage 0 began at the top of the unit
        if (!active) continue;
        const int kc = W_FP8 ? r : r >> 1;
        const u16* ukc = us + kc * UROWS * kChunk;
        const u16* wbuf = ws + (g & 1) * Tile::RING_ELEMS;
        if constexpr (W_FP8) {
          // the lane's 8 weights of a tap: 8 bytes, widened when read
          conv_stage(std::integral_constant<int, kTaps>{},
                     wbuf + (wco0 + lrow) * Tile::P_LO * 8 + lk / 2, ukc, 0);
        } else {
          // bf16 weights (taps 0-3 or 4-6 of the chunk; the lane's 8 weights of a tap: 16
          // bytes): one loop over the stage's taps, each reading its TP operand tiles and TCO
          // weight tiles before its first MFMA, one LDS wait per tap (the pipelined stage above
          // needs more registers than two waves per SIMD have with bf16 weights: 256 VGPRs and
          // 368 bytes of spills)
          const int t0 = (r & 1) ? 4 : 0;
          const int nt = (r & 1) ? 3 : 4;
          constexpr int P8 = Tile::P_LO * 8;  // u16 elements per weight row
          // tap jj's slot 4 jj + lane / 16 of column row n sits at (4 jj + lane / 16) ^ (n % 16),
          // and n % 16 = lrow in every column tile
          const u16* wrow = wbuf + (wco0 + lrow) * P8;
          const int wq = ((lane >> 4) ^ lrow) & 3;
          const int wt = lrow >> 2;
#pragma unroll 1
          for (int jj = 0; jj < nt; ++jj) {
            const int rj = row0 + (t0 + jj) * d - h;
            const int bj = rj * kChunk + (((lane >> 4) ^ ((rj >> 1) & 3)) << 3);
            bf16x8 bv[TP], a[TCO];
#pragma unroll
            for (int t = 0; t < TP; ++t)
              bv[t] = *reinterpret_cast<const bf16x8*>(ukc + bj + t * 16 * kChunk);
            const u16* wtap = wrow + ((((jj ^ wt) << 2) | wq) << 3);
#pragma unroll
            for (int c = 0; c < TCO; ++c) a[c] = *reinterpret_cast<const bf16x8*>(wtap + c * 16 * P8);
#pragma unroll
            for (int c = 0; c < TCO; ++c)
#pragma unroll
              for (int t = 0; t < TP; ++t)
                acc[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c], bv[t], acc[c][t], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, TP + TCO, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, TP * TCO, 0);
          }
        }
      }
    }
    // every wave's reads of the operand tile (its rows are other waves' halo) and of the last
    // conv stage's weights are done before h overwrites the tile: the k = 1 weights' stage
    // barrier (its DMA ran during the last conv stage) is that point
    const int g2 = k * Tile::STAGES + Tile::CONV_STAGES;
    stage_begin(g2);
    const u16* w2s = ws + (g2 & 1) * Tile::RING_ELEMS;
    if (active) {
    // (d) h = Snake(acc * scale + bias) over the operand tile; the k = 1 weights
    const float* cf = coef + k * kCoefRows * C;
#pragma unroll
    for (int c = 0; c < TCO; ++c) {
      const int n = wco0 + c * 16 + (lane >> 4) * 4;
      const f32x4 sc = *reinterpret_cast<const f32x4*>(cf + kS1 * C + n);
      const f32x4 bi = *reinterpret_cast<const f32x4*>(cf + kB1 * C + n);
      const f32x4 ma = *reinterpret_cast<const f32x4*>(cf + kMA * C + n);
      const f32x4 mb = *reinterpret_cast<const f32x4*>(cf + kMB * C + n);
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = operand_act(OMNI_ACT_SNAKE, acc[c][t][e] * sc[e] + bi[e], ma[e], mb[e], 0.f);
        put(c, t, y[0], y[1], y[2], y[3]);
        acc[c][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    // (e) the k = 1 conv; it reads only the rows this wave wrote in (d), so no barrier is needed
    // between them (LDS operations of one wave complete in order)
#pragma unroll
    for (int kc = 0; kc < CH; ++kc) {
      bf16x8 a[TCO];
#pragma unroll
      for (int c = 0; c < TCO; ++c) {
        const int row = kc * C + wco0 + c * 16 + lrow;
        if constexpr (W_FP8)  // the ring holds the E4M3 bytes: 32 per row
          a[c] = __builtin_bit_cast(bf16x8, fp8x8_to_bf16x8(*reinterpret_cast<const u32x2*>(
                                                w2s + row * (kChunk / 2) + lk / 2)));
        else  // slot lane / 16 of row `row` at (lane / 16) ^ ((row / 2) % 4)
          a[c] = *reinterpret_cast<const bf16x8*>(
              w2s + row * kChunk + ((((lane >> 4) ^ (row >> 1)) & 3) << 3));
      }
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(
            us + rd_base + kc * UROWS * kChunk + t * 16 * kChunk);
#pragma unroll
        for (int c = 0; c < TCO; ++c)
          acc[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c], bv, acc[c][t], 0, 0, 0);
      }
    }
    // (f) overwrites only this wave's rows of the tile, which no other wave reads in (e), and the
    // k = 1 weights' buffer is next written after the next unit's first stage barrier: no
    // barrier here
    // (f) x += acc * scale + bias; the next operand Snake(x) (the next unit's input Snake, or
    // the output Snake)
#pragma unroll
    for (int c = 0; c < TCO; ++c) {
      const int n = wco0 + c * 16 + (lane >> 4) * 4;
      const f32x4 sc = *reinterpret_cast<const f32x4*>(cf + kS2 * C + n);
      const f32x4 bi = *reinterpret_cast<const f32x4*>(cf + kB2 * C + n);
      const f32x4 na = *reinterpret_cast<const f32x4*>(cf + kNA * C + n);
      const f32x4 nb = *reinterpret_cast<const f32x4*>(cf + kNB * C + n);
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        f32x4 v = acc[c][t] * sc + bi;
        v += xv[c][t];
        xv[c][t] = v;
        put(c, t, snake_rev(v[0], na[0], nb[0]), snake_rev(v[1], na[1], nb[1]),
            snake_rev(v[2], na[2], nb[2]), snake_rev(v[3], na[3], nb[3]));
      }
    }
    }  // active
    halo_move(k + 1);
  }
  // In the sweep, the next tile's x (no halo rows ahead of it) is loaded now, while this tile's
  // final conv and output stores run, instead of at the start of the next tile where the first
  // operand waits for it; only when x_last is not stored, so the residual stream is free.
  x_ready = false;
  if constexpr (SWEEP) {
    if (has_next && p.x_out == nullptr) {
      const int ni0 = i0 + len;
      const int nrows = min(Tile::R, seg_end - ni0);
      const auto xr = buffer_rsrc(p.x, p.x_bytes);
      const int ln = opaque_copy(lane);
#pragma unroll
      for (int c = 0; c < TCO; ++c) {
        const int n = wco0 + c * 16 + (ln >> 4) * 4;
#pragma unroll
        for (int t = 0; t < TP; ++t) {
          const int r = wave_p * TP * 16 + t * 16 + (ln & 15);
          const int pos = ni0 + r;
          const bool ok = r < nrows && pos < L;
          const uint32_t off = ok ? (uint32_t)(b0 * p.x_sb + pos * p.x_st + n) * xsize : kOutOfRange;
          // the raw bits (a float16 stream in the first two words), widened where the next tile
          // first reads them, so this load's wait stays there
          xv[c][t] = __builtin_bit_cast(f32x4, omni_conv::load_residual4_raw(xr, off, p.x_f16));
        }
      }
      x_ready = true;
    }
  }
  __syncthreads();
  // ---- the output operand rows of the tile's positions, 16 contiguous bytes per thread
  if (p.out != nullptr) {
    const auto orsrc = buffer_rsrc(p.out, p.o_bytes);
    for (int e = opaque_copy(tid); e < nseg * len * PIECES_PER_ROW; e += NT) {
      const int s = e / (len * PIECES_PER_ROW);
      const int rem = e - s * len * PIECES_PER_ROW;
      const int q = rem / PIECES_PER_ROW;
      const int piece = rem - q * PIECES_PER_ROW;
      const int row = GUARD + s * span + H + q;
      const u32x4 v = *reinterpret_cast<const u32x4*>(us + uaddr<UROWS>(piece >> 2, row, piece & 3));
      const uint32_t off = (uint32_t)((b0 + s) * p.o_sb + (i0 + q) * p.o_st + piece * 8) * 2;
      __builtin_amdgcn_raw_buffer_store_b128(v, orsrc, off, 0, 0);
    }
  }
  // ---- the decoder's final conv to one channel over the output operand u in LDS, in the
  // summation order of single_output_conv_bf16_kernel (j outer, channels ascending, one fma each)
  if (p.fin_w != nullptr) {
    const int fh = p.fin_taps - 1;  // its causal context: staged rows H - fh .. H - 1
    const auto fr = buffer_rsrc(p.fin_hist, p.fin_hist_bytes);
    // (a) context rows left of position 0 (segments that start a stream row): the history copy
    // of the row's slot, or zeros
    if (i0 == 0 && fh > 0) {
      for (int e = opaque_copy(tid); e < nseg * fh * PIECES_PER_ROW; e += NT) {
        const int s = e / (fh * PIECES_PER_ROW);
        const int rem = e - s * fh * PIECES_PER_ROW;
        const int j = rem / PIECES_PER_ROW;  // sample j of the history: position j - fh
        const int piece = rem - j * PIECES_PER_ROW;
        uint32_t off = kOutOfRange;
        if (p.fin_hist != nullptr && !p.hist_cold) {
          const int64_t slot = p.slot_index[b0 + s];
          if (slot >= 0 && slot < p.hist_slots) {
            const int parity = (int)(p.slot_parity[slot] & 1);
            off = (uint32_t)((int)slot * p.fin_hist_stride + (parity * fh + j) * C + piece * 8) * 2;
          }
        }
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(fr, off, 0, 0);
        const int row = GUARD + s * span + H - fh + j;
        *reinterpret_cast<u32x4*>(us + uaddr<UROWS>(piece >> 2, row, piece & 3)) = v;
      }
    }
    __syncthreads();
    // (b) its new history: the last fh operand samples of each stream row, written by the
    // workgroup holding them (those left of 0 by the one holding position 0); as the units', only
    // in a tile that holds a row's last fh positions or its start
    if (p.fin_hist != nullptr && (i0 == 0 || i0 + len > L - fh)) {
      for (int e = opaque_copy(tid); e < nseg * fh * PIECES_PER_ROW; e += NT) {
        const int s = e / (fh * PIECES_PER_ROW);
        const int rem = e - s * fh * PIECES_PER_ROW;
        const int j = rem / PIECES_PER_ROW;
        const int piece = rem - j * PIECES_PER_ROW;
        const int pos = L - fh + j;
        const bool own = pos >= 0 ? (pos >= i0 && pos < i0 + len) : i0 == 0;
        const int64_t slot = p.slot_index[b0 + s];
        if (own && slot >= 0 && slot < p.hist_slots) {
          const int parity = (int)(p.slot_parity[slot] & 1);
          const int row = GUARD + s * span + (pos - i0) + H;
          const u32x4 v = *reinterpret_cast<const u32x4*>(us + uaddr<UROWS>(piece >> 2, row, piece & 3));
          const uint32_t off =
              (uint32_t)((int)slot * p.fin_hist_stride + ((1 - parity) * fh + j) * C + piece * 8) * 2;
          __builtin_amdgcn_raw_buffer_store_b128(v, fr, off, 0, 0);
        }
      }
    }
    // (c) the conv on the matrix cores with the taps as the columns: column j of the A operand
    // holds tap j's weights (fin_a), the B operand is the operand tile at the rows' own
    // positions, so one MFMA per 32-channel chunk and 16 rows gives D[j][row] = sum_c w[j][c]
    // u[row][c] for every tap; then out[row] = sum_j D[j][row - fh + j] (taps ascending) + bias,
    // from D through LDS ([16 + R][8] floats in the ring, which is free now). Wave 0 also
    // computes the 16 rows ahead of row 0 (the guard, where the sweep keeps the previous tile's
    // last operand rows).
    float* dl = reinterpret_cast<float*>(ws);
    static_assert((16 + Tile::R) * 8 * 4 <= Tile::W_ELEMS * 2, "D fits the ring");
    const int ln = opaque_copy(lane);
    f32x4 dg = f32x4{0.f, 0.f, 0.f, 0.f};  // wave 0: the guard rows -16 .. -1
#pragma unroll
    for (int t = 0; t < TP; ++t) acc[0][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    {
      const int rt = GUARD + wave_p * TP * 16 + (ln & 15);
      const int bt = rt * kChunk + (((ln >> 4) ^ ((rt >> 1) & 3)) << 3);
      const int rg = GUARD - 16 + (ln & 15);
      const int bg = rg * kChunk + (((ln >> 4) ^ ((rg >> 1) & 3)) << 3);
#pragma unroll
      for (int kc = 0; kc < CH; ++kc) {
        const bf16x8 a = fin_a[kc];
        const u16* ukc = us + kc * UROWS * kChunk;
#pragma unroll
        for (int t = 0; t < TP; ++t) {
          const bf16x8 bv = *reinterpret_cast<const bf16x8*>(ukc + bt + t * 16 * kChunk);
          acc[0][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bv, acc[0][t], 0, 0, 0);
        }
        if (wave_p == 0) {
          const bf16x8 bv = *reinterpret_cast<const bf16x8*>(ukc + bg);
          dg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bv, dg, 0, 0, 0);
        }
      }
    }
    // lane l holds D[4 (l / 16) + e][row l % 16 of the block]: taps 0..7 in lanes 0..31
    if ((ln >> 4) < 2) {
#pragma unroll
      for (int t = 0; t < TP; ++t)
        *reinterpret_cast<f32x4*>(dl + (16 + row_of(t, ln & 15)) * 8 + (ln >> 4) * 4) = acc[0][t];
      if (wave_p == 0) *reinterpret_cast<f32x4*>(dl + (ln & 15) * 8 + (ln >> 4) * 4) = dg;
    }
    __syncthreads();
    const float bias = p.fin_b ? p.fin_b[0] : 0.f;
    for (int r = opaque_copy(tid); r < rows; r += NT) {
      const int sg = SWEEP ? 0 : r / span;
      const int q = r - sg * span;
      if (q >= H) {
        const float* dr = dl + (16 + r - fh) * 8;
        float v = dr[0];
        for (int j = 1; j <= fh; ++j) v += dr[j * 8 + j];
        p.fin_out[(int64_t)(b0 + sg) * p.fin_o_sb + (i0 - H + q)] =
            apply_act(p.fin_act, v + bias, 0.f, 0.f, 0.f);
      }
    }
  }
  if (p.x_out != nullptr) {
    const auto xo = buffer_rsrc(p.x_out, p.xo_bytes);
    const int ln = opaque_copy(lane);
    const int lr = ln & 15;
#pragma unroll
    for (int c = 0; c < TCO; ++c) {
      const int n = wco0 + c * 16 + (ln >> 4) * 4;
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const int q = row_of(t, lr) - seg_of(t, lr) * span;
        const bool ok = row_of(t, lr) < rows && q >= H;
        const uint32_t off =
            ok ? (uint32_t)((b0 + seg_of(t, lr)) * p.xo_sb + pos_of(t, lr) * p.xo_st + n) * xsize
               : kOutOfRange;
        omni_conv::store_residual4(xv[c][t], xo, off, p.x_f16);
      }
    }
  }
  if (!has_next) break;
  i0 += len;
  }  // tiles
}

// 96 channels, 8 waves, each with all 96 columns and 48 of the 384 staged rows (the register
// budget of two waves per SIMD: x and the accumulators); bf16 or E4M3 weights by LDS DMA.
using Stack96Dma = StackTile<96, 1, 8, 3>;
using Stack96Sweep = StackTile<96, 1, 8, 3, true>;
using Stack96Dma8 = StackTile<96, 1, 8, 3, false, true>;
using Stack96Sweep8 = StackTile<96, 1, 8, 3, true, true>;
static_assert(Stack96Sweep::lds_bytes() <= 160 * 1024, "the sweep form fits the CU's LDS");
static_assert(Stack96Sweep8::lds_bytes() <= Stack96Sweep::lds_bytes() &&
              Stack96Dma8::R == Stack96Dma::R && Stack96Sweep8::R == Stack96Dma::R,
              "E4M3 weights take the bf16 forms' tiles");

template <bool W_FP8>
int launch_stack96(const StackParams& p, int grid, bool sweep, hipStream_t stream);
template <> int launch_stack96<false>(const StackParams& p, int grid, bool sweep, hipStream_t stream);
template <> int launch_stack96<true>(const StackParams& p, int grid, bool sweep, hipStream_t stream);

}  // namespace omni_stack
