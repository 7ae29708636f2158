// The fused residual unit (conv k7 -> Snake -> conv k1 -> + x) with LDS-DMA staging, for
// 192-channel layers with bf16 weights whose operand is a ready bf16 activation (gfx950 bf16
// MFMA). (With E4M3 weights the register-staged fused form is faster: widening the weight bytes
// on the operand read costs this kernel registers it does not have.)
//
// conv_mfma_kernel's fused form (conv_kernel.h, FUSE2) stages each 32-channel chunk of the
// operand and of the k7 weights through registers: per wave four times as many VALU as MFMA
// instructions. Here the operand rows and the weights reach LDS by DMA (buffer_load ... lds), as
// in conv_dma_kernel (conv_dma.h), whose input staging (row segments with their own halo, history
// rows left of position 0, the new history written from LDS, causal zero rows) this kernel
// repeats. One column tile holds all 192 channels, since the k1 conv needs every channel of h: a
// chunk's weights for 192 columns and 7 taps (89 KB) would not double-buffer, so a ring stage
// holds taps 0-3 or 4-6 of a chunk's weights, two stages per chunk, and each ring buffer also
// holds the input rows of every other chunk (chunk kc in buffer kc % 2, staged once for both of
// its stages).
// After the last stage the W2 weights (DMA'd into the free ring buffer during it) and h =
// Snake(acc * scale + bias) (into the other) feed the k1 conv, whose accumulators go through
// conv_epilogue (residual, float32 residual stream, the next operand's activation).
//
// Every accumulator takes its MFMAs in the order of conv_mfma_kernel's fused form (chunks, then
// taps; the k1 conv by chunks), h rounds the same way and the epilogue is shared, so the two
// kernels give the same bits.
#pragma once

#include "conv_dma.h"

namespace omni_conv {

struct FusedDmaTile {
  static constexpr int WAVES_CO = 2, WAVES_P = 4, TCO = 6, TP = 3;
  static constexpr int MAX_ROWS = 192 + 2 * kMaxHalo;
  using Base = ConvTile<WAVES_CO, WAVES_P, TCO, TP, MAX_ROWS, 7>;  // epilogue geometry
  static constexpr int NT = Base::NT;
  static constexpr int BCO = Base::BCO;  // 192: every channel
  static constexpr int BP = Base::BP;    // 192 positions
  static constexpr int NW = NT / 64;
  static constexpr int CH = BCO / kChunk;
  // 16-byte slots per weight row of a 4-tap / 3-tap stage, plus two pad slots: a pitch of 2 mod 4
  // slots, at which the 16 column rows of an MFMA operand read meet no LDS bank conflict
  static constexpr int P4 = 4 * 4 + 2;
  static constexpr int P3 = 3 * 4 + 2;
  static constexpr int NIW4 = (BCO * P4 + 63) / 64;  // weight DMA instructions of a stage
  static constexpr int NIW3 = (BCO * P3 + 63) / 64;
  static constexpr int W4_PIECES = (NIW4 + NW - 1) / NW;
  static constexpr int W3_PIECES = (NIW3 + NW - 1) / NW;
  static constexpr int NIX = MAX_ROWS / 16;  // input-row DMA instructions of a stage
  static constexpr int X_PIECES = (NIX + NW - 1) / NW;
  static constexpr int XCHUNK = MAX_ROWS * kChunk;  // elements of a stage's input rows
  static constexpr int WSTAGE = NIW4 * 64 * 8;      // elements of a stage's weights
  static constexpr int W2_ELEMS = CH * BCO * kChunk;  // W2 in LDS
  static constexpr int NIW2 = W2_ELEMS * 2 / 16 / 64;
  static constexpr int W2_PIECES = (NIW2 + NW - 1) / NW;
  static constexpr int H_ELEMS = CH * BP * kChunk;
  // a ring buffer: a stage, then W2 or h
  static constexpr int BUF = XCHUNK + WSTAGE > H_ELEMS ? XCHUNK + WSTAGE : H_ELEMS;
  static constexpr size_t ring_bytes = 2 * (size_t)BUF * 2;
  static constexpr size_t epi_bytes = (size_t)Base::EPI_ROWS * Base::EPITCH * 4;
  static constexpr size_t coef_offset = ring_bytes > epi_bytes ? ring_bytes : epi_bytes;
  static constexpr size_t lds_bytes = coef_offset + Base::coef_bytes();
  static_assert(NIW2 * 64 * 16 == W2_ELEMS * 2, "W2 is whole DMA instructions");
  static_assert(W2_ELEMS <= BUF && H_ELEMS <= BUF, "W2 and h each fit a ring buffer");
  static_assert(X_PIECES <= 16, "two mode bits per input piece in 32 bits");
  static_assert(lds_bytes <= 160 * 1024, "the ring, epilogue and coefficients fit the CU's LDS");
};

// (internal linkage: the header reaches more than one translation unit, and only the bf16
// fused launcher launches it)
static __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
    fused_unit_dma_kernel(const ConvParams p) {
  using Tile = FusedDmaTile;
  constexpr int NT = Tile::NT;
  constexpr int NW = Tile::NW;
  constexpr int BCO = Tile::BCO;
  constexpr int BP = Tile::BP;
  constexpr int TCO = Tile::TCO;
  constexpr int TP = Tile::TP;
  constexpr int CH = Tile::CH;
  constexpr int MAX_ROWS = Tile::MAX_ROWS;
  constexpr int WAVES_CO = Tile::WAVES_CO;
  extern __shared__ __attribute__((aligned(16))) u16 lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wave_co = wave % WAVES_CO;
  const int wave_p = wave / WAVES_CO;
  const int p_tile = xcd_tile(blockIdx.x, gridDim.x);

  const int dil = p.dil;
  const int lpad = p.lpad;
  const int halo = p.halo;
  const int L = p.length;
  const int XL = p.x_length;
  const int H = lpad;

  // The tile's positions [m0, m_end) of the flattened (row, position) space and its row segments
  const int M = p.batch * L;
  const int m0 = p_tile * BP;
  const int m_end = min(m0 + BP, M);
  const int b0 = m0 / L;
  const int lo0 = m0 - b0 * L;
  const int first = min(L - lo0, m_end - m0);
  const int nseg = (m_end - 1) / L - b0 + 1;
  const int rows = (m_end - m0) + nseg * halo;
  const int seg_rows = L + halo;

  // Input-row DMA descriptors, as conv_dma_kernel's but with the quarters in order (the swizzle's
  // address arithmetic on every operand read costs this kernel registers it does not have):
  // piece u of thread tid is staged row r = tid / 4 + u * NT / 4, quarter tid % 4; its element
  // offset at channel q8 of chunk 0 in x or in the history pool, its source (2 bits: 0 zeros,
  // 1 x, 2 history, 3 not staged) and, when it is a sample of the new history this workgroup
  // writes, its offset there.
  const int q8 = (tid & 3) * 8;
  int xoff[Tile::X_PIECES];
  int hwoff[Tile::X_PIECES];
  unsigned xmode = 0;
  const bool may_write_history = p.hist != nullptr && H > 0;
#pragma unroll
  for (int u = 0; u < Tile::X_PIECES; ++u) {
    const int r = (tid >> 2) + u * (NT / 4);
    const int lq8 = q8;
    int off = 0;
    int hw = -1;
    unsigned mode = 3;
    if (r < rows && r < MAX_ROWS) {
      mode = 0;
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
        off = (int)(b * p.x_sb + (int64_t)pos * p.x_st) + lq8;
        mode = 1;
      } else if (pos < 0 && slot >= 0 && !p.hist_cold) {
        off = (int)(slot * p.hist_slot_stride + (parity * H + (H + pos)) * (int64_t)BCO) + lq8;
        mode = 2;
      }
      if (may_write_history && slot >= 0 && pos >= XL - H && pos < XL) {
        const int64_t m = (int64_t)b * L + pos;
        const bool owned = pos >= 0 ? (m >= m0 && m < m_end) : row_start;
        if (owned)
          hw = (int)(slot * p.hist_slot_stride + ((1 - parity) * H + (pos - (XL - H))) *
                                                     (int64_t)BCO) + lq8;
      }
    }
    xoff[u] = off;
    hwoff[u] = hw;
    xmode |= mode << (2 * u);
  }

  // Weight DMA descriptors of the two stage patterns: slot s = 64 * (wave + u * NW) + lane of a
  // stage's weight area is column s / P, piece s % P (the last piece is the pad). The packed
  // weights of chunk kc are [n_cols][7][32]: column n's taps t0.. start at byte
  // ((kc * n_cols + n) * 7 + t0) * 64, so the per-lane part (n * 7 * 64 + piece * 16)
  // is the same for every chunk and tap start.
  uint32_t woff4[Tile::W4_PIECES], woff3[Tile::W3_PIECES];
  {
    auto slot_offset = [&](int di, int P, int nt) __attribute__((always_inline)) {
      const int s = di * 64 + lane;
      const int n = s / P;
      const int piece = s - n * P;
      return (n < BCO && piece < nt * 4) ? (uint32_t)(n * 7 * kChunk * 2 + piece * 16) : 0u;
    };
#pragma unroll
    for (int u = 0; u < Tile::W4_PIECES; ++u) woff4[u] = slot_offset(wave + u * NW, Tile::P4, 4);
#pragma unroll
    for (int u = 0; u < Tile::W3_PIECES; ++u) woff3[u] = slot_offset(wave + u * NW, Tile::P3, 3);
  }

  float* coef = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(lds) + Tile::coef_offset);
  stage_coefficients<BCO, NT, true>(p, coef, 0);

  auto buf_of = [&](int b) __attribute__((always_inline)) -> u16* { return lds + b * Tile::BUF; };

  // Zero padding rows: written once into both buffers (no DMA writes them).
#pragma unroll
  for (int u = 0; u < Tile::X_PIECES; ++u) {
    if (((xmode >> (2 * u)) & 3u) == 0u) {
      const int r = (tid >> 2) + u * (NT / 4);
      for (int b = 0; b < 2; ++b)
        *reinterpret_cast<u32x4*>(buf_of(b) + r * kChunk + q8) = u32x4{0u, 0u, 0u, 0u};
    }
  }

  const auto x_rsrc = buffer_rsrc(p.x, p.x_bytes);
  const auto h_rsrc = buffer_rsrc(p.hist, p.hist_bytes);
  const auto w_rsrc = buffer_rsrc(p.weight, p.w_bytes);
  const auto w2_rsrc = buffer_rsrc(p.weight2, p.w2_bytes);
  typedef __attribute__((address_space(3))) void* lds_ptr_t;

  // Stage s: chunk kc = s / 2, taps 0-3 (s even) or 4-6 (s odd): the taps' weights into ring
  // buffer s % 2 and, for the chunk's first stage, its input rows into buffer kc % 2 (where both
  // of the chunk's stages read them: the other chunk's rows there were last read two stages back).
  auto issue = [&](int s) __attribute__((always_inline)) {
    const int kc = s >> 1;
    const int g = s & 1;
    u16* xs = buf_of(kc & 1);
    u16* ws = buf_of(s & 1) + Tile::XCHUNK;
    const uint32_t wbase = (uint32_t)((kc * p.n_cols * 7 + g * 4) * kChunk * 2);
    if (g == 0) {
#pragma unroll
      for (int u = 0; u < Tile::W4_PIECES; ++u) {
        const int iw = wave + u * NW;
        if (iw < Tile::NIW4)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(ws + iw * 64 * 8), 16,
                                                   (int)woff4[u], (int)wbase, 0, 0);
      }
    } else {
#pragma unroll
      for (int u = 0; u < Tile::W3_PIECES; ++u) {
        const int iw = wave + u * NW;
        if (iw < Tile::NIW3)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(ws + iw * 64 * 8), 16,
                                                   (int)woff3[u], (int)wbase, 0, 0);
      }
    }
    if (g != 0) return;
    const uint32_t xbase = (uint32_t)(kc * kChunk * 2);
#pragma unroll
    for (int u = 0; u < Tile::X_PIECES; ++u) {
      const int ii = wave + u * NW;
      if (ii < Tile::NIX) {
        const unsigned mode = (xmode >> (2 * u)) & 3u;
        lds_ptr_t dst = (lds_ptr_t)(xs + ii * 64 * 8);
        if (mode == 1u)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rsrc, dst, 16, (int)((uint32_t)xoff[u] * 2u),
                                                   (int)xbase, 0, 0);
        else if (mode == 2u)  // with the non-temporal hint (aux 2), which keeps the compiler
                              // from merging the two DMAs into one whose buffer descriptor
                              // differs between lanes (a readfirstlane loop)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(h_rsrc, dst, 16, (int)((uint32_t)xoff[u] * 2u),
                                                   (int)xbase, 0, 2);
      }
    }
  };
  // W2 ([C/32][C][32] as stored) into ring buffer b: 64-byte rows, slot s of row r holding the
  // row's piece s ^ ((r / 2) % 4)
  auto issue_w2 = [&](int b) __attribute__((always_inline)) {
    u16* w2s = buf_of(b);
#pragma unroll
    for (int u = 0; u < Tile::W2_PIECES; ++u) {
      const int iw = wave + u * NW;
      const int slot = iw * 64 + lane;
      if (iw < Tile::NIW2)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w2_rsrc, (lds_ptr_t)(w2s + iw * 64 * 8), 16,
                                                 (int)((uint32_t)(slot ^ ((slot >> 3) & 3)) * 16u),
                                                 0, 0, 0);
    }
  };
  // The new history samples of chunk kc (its input rows in buffer b), from LDS to the slot's
  // other copy.
  auto write_history = [&](int kc, int b) __attribute__((always_inline)) {
    const u16* xs = buf_of(b);
#pragma unroll
    for (int u = 0; u < Tile::X_PIECES; ++u) {
      if (hwoff[u] >= 0) {
        const int r = (tid >> 2) + u * (NT / 4);
        const u32x4 v = *reinterpret_cast<const u32x4*>(xs + r * kChunk + q8);
        __builtin_amdgcn_raw_buffer_store_b128(v, h_rsrc, (uint32_t)(hwoff[u] + kc * kChunk) * 2,
                                               0, 0);
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
  int xrow[TP];  // this lane's staged row for each of its position groups (tap 0)
#pragma unroll
  for (int t = 0; t < TP; ++t) {
    const int m = m0 + wp0 + t * 16 + lrow;
    xrow[t] = m < m_end ? (m - m0) + (m / L - b0) * halo : 0;
  }

  // ---- the k7 conv: 2 * CH stages, one barrier each; the next stage's DMA runs under this
  // stage's MFMAs, and W2's under the last stage's
  constexpr int STAGES = 2 * CH;
  issue(0);
  for (int s = 0; s < STAGES; ++s) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (s + 1 < STAGES) issue(s + 1);
    else issue_w2((s + 1) & 1);
    if (p.hist != nullptr && (s & 1) == 0) write_history(s >> 1, (s >> 1) & 1);
    const int g = s & 1;
    const int t0 = g * 4;
    const u16* xs = buf_of((s >> 1) & 1);         // the chunk's input rows
    const u16* wsb = buf_of(s & 1) + Tile::XCHUNK;  // the stage's weights
    // the stage's taps, software-pipelined: tap i + 1's operands are read from LDS before tap
    // i's MFMAs
    auto stage_taps = [&](auto ntc) __attribute__((always_inline)) {
      constexpr int NTAPS = decltype(ntc)::value;
      constexpr int P8 = (NTAPS == 4 ? Tile::P4 : Tile::P3) * 8;  // u16 elements per weight row
      auto load_tap = [&](int i, bf16x8 (&a)[TCO], bf16x8 (&bv)[TP]) __attribute__((always_inline)) {
        const u16* wtap = wsb + (wco0 + lrow) * P8 + lk + i * kChunk;
#pragma unroll
        for (int cc = 0; cc < TCO; ++cc)
          a[cc] = *reinterpret_cast<const bf16x8*>(wtap + cc * 16 * P8);
        const int shift = (t0 + i) * dil;
#pragma unroll
        for (int t = 0; t < TP; ++t)
          bv[t] = *reinterpret_cast<const bf16x8*>(xs + (xrow[t] + shift) * kChunk + lk);
      };
      bf16x8 a[2][TCO], bv[2][TP];
      load_tap(0, a[0], bv[0]);
#pragma unroll
      for (int i = 0; i < NTAPS; ++i) {
        if (i + 1 < NTAPS) load_tap(i + 1, a[(i + 1) & 1], bv[(i + 1) & 1]);
#pragma unroll
        for (int t = 0; t < TP; ++t)
#pragma unroll
          for (int cc = 0; cc < TCO; ++cc)
            acc[cc][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i & 1][cc], bv[i & 1][t],
                                                                 acc[cc][t], 0, 0, 0);
      }
    };
    if (g == 0) stage_taps(std::integral_constant<int, 4>{});
    else stage_taps(std::integral_constant<int, 3>{});
  }

  // ---- h = mid_act(acc * scale + bias) as bf16 into ring buffer (STAGES - 1) % 2 once every
  // wave's reads of the last stage are done: [CH][BP][32], the four 16-byte slots of a 64-byte
  // row rotated by (row / 4) % 4 (as conv_mfma_kernel's fused form lays it out)
  const int ch_in_tile = (lane >> 4) * 4;
  u16* hs = buf_of((STAGES - 1) & 1);
  const u16* w2s = buf_of(STAGES & 1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's W2 DMA
  __syncthreads();
  // (the activation a compile-time constant of each copy: one branch for the whole tile)
  auto put_h = [&](auto act_c) __attribute__((always_inline)) {
    constexpr int ACT = decltype(act_c)::value;
#pragma unroll
    for (int c = 0; c < TCO; ++c) {
      const int n = wco0 + c * 16 + ch_in_tile;
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
  else if (p.mid_act == OMNI_ACT_LEAKY_RELU) put_h(std::integral_constant<int, OMNI_ACT_LEAKY_RELU>{});
  else put_h(std::integral_constant<int, OMNI_ACT_NONE>{});
  __syncthreads();  // h complete, W2 visible to every wave
  // ---- the k1 conv over h
#pragma unroll
  for (int kc = 0; kc < CH; ++kc) {
    bf16x8 a[TCO];
#pragma unroll
    for (int c = 0; c < TCO; ++c) {
      const int row = kc * BCO + wco0 + c * 16 + lrow;
      a[c] = *reinterpret_cast<const bf16x8*>(w2s + row * kChunk +
                                              ((((lane >> 4) ^ (row >> 1)) & 3) << 3));
    }
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

  // (no mix: the launcher refuses it)
  conv_epilogue<typename Tile::Base, Tile::WAVES_P, TCO, TP, false>(p, acc, lds, coef, kScale2,
                                                                    kBias2, 0, m0, m_end, wave_p,
                                                                    wco0);
}

struct FusedDmaConfig {
  using Tile = FusedDmaTile;

  // Staged rows of the fullest tile: BP positions over at most nseg row segments, each with its
  // own halo.
  static int64_t rows_needed(const ConvParams& p) {
    const int64_t bp = Tile::BP;
    int64_t nseg = (bp + p.length - 2) / p.length + 1;
    if (nseg > p.batch) nseg = p.batch;
    return bp + nseg * p.halo;
  }

  // A 192-channel unit (k7 conv of C_in = C_out = 192, then the k1 conv 192 -> 192) whose staged
  // rows fit, with no mix in its epilogue (the register-staged kernels take that).
  static bool fits(const ConvParams& p) {
    return p.taps == 7 && p.n_cols == Tile::BCO && p.c_out == Tile::BCO && p.c_in == Tile::BCO &&
           p.weight2 != nullptr && p.mix_a == nullptr && rows_needed(p) <= Tile::MAX_ROWS;
  }

  static int64_t workgroups(const ConvParams& p) {
    return ((int64_t)p.batch * p.length + Tile::BP - 1) / Tile::BP;
  }

  static int launch(ConvParams p, hipStream_t stream) {
    p.p_tiles = (int)workgroups(p);
    p.n_tiles = 1;
    auto k = fused_unit_dma_kernel;
    static const bool raised = raise_lds_limit((const void*)k);
    (void)raised;
    hipLaunchKernelGGL(k, dim3((unsigned)p.p_tiles), dim3(Tile::NT), Tile::lds_bytes, stream, p);
    OMNI_LAUNCH_CHECK();
    return OMNI_OK;
  }
};

}  // namespace omni_conv

namespace omni_conv {

// The fused residual-unit list of one channel count: the LDS-DMA tile (192 channels, bf16
// weights and operands as they are; `Dma` = void elsewhere), then the register-staged full tile and its
// short-row tile (entries 1, 2 and 3 of a forced choice). The first that fits runs.
template <bool W_FP8, typename Dma, typename Full, typename Short>
int launch_fused_list(const ConvParams& p, int in_mode, Choice& ch, hipStream_t stream) {
  bool dma_fits = false;
  int64_t dma_wgs = 0;
  int (*dma_run)(ConvParams, hipStream_t) = nullptr;
  if constexpr (!std::is_void<Dma>::value) {
    dma_fits = in_mode == IN_RAW && Dma::fits(p);
    dma_wgs = Dma::workgroups(p);
    dma_run = &Dma::launch;
  }
  const bool fits[3] = {dma_fits, Full::fits(p, true), Short::fits(p, true)};
  const int64_t wgs[3] = {dma_wgs, Full::workgroups(p), Short::workgroups(p)};
  int (*run[3])(ConvParams, hipStream_t);
  run[0] = dma_run;
  if (in_mode == IN_RAW) {
    run[1] = &Full::template launch<IN_RAW, W_FP8, true>;
    run[2] = &Short::template launch<IN_RAW, W_FP8, true>;
  } else if (in_mode == IN_ACT) {
    run[1] = &Full::template launch<IN_ACT, W_FP8, true>;
    run[2] = &Short::template launch<IN_ACT, W_FP8, true>;
  } else {
    run[1] = &Full::template launch<IN_F32, W_FP8, true>;
    run[2] = &Short::template launch<IN_F32, W_FP8, true>;
  }
  const int pick = fits[0] ? 0 : (fits[1] ? 1 : (fits[2] ? 2 : -1));
  return choose_and_launch(ch, 3, fits, wgs, run, pick, p, stream);
}

}  // namespace omni_conv
