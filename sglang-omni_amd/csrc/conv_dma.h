// Polyphase convolution with LDS-DMA staging (gfx950 bf16 MFMA), for bf16 operands used as they
// are (no activation on the way in) and bf16 or E4M3 weights: the conv layers of the codec
// decoder, whose producers write the next conv's operand u = act(x) from their epilogues.
//
// The GEMM is conv_mfma_kernel's (conv_kernel.h): output columns n as the MFMA M dimension,
// positions m = b * length + i as N, (tap, c_in) as K, batch rows sharing one position space with
// a (taps-1)*dil halo staged per row segment. What differs is how the operands reach LDS:
//
//   * Buffer loads with the LDS-DMA bit (buffer_load_dwordx4 ... lds) move each 16-byte piece
//     from HBM straight into LDS: no staging registers, no LDS store instructions, and the waves
//     issue a stage's loads in a few instructions. Lane l of a DMA instruction fills the 16-byte
//     LDS slot 64 * instr + l, so each lane loads the piece that belongs in its slot:
//       - input rows [rows][32] (64-byte rows): instruction ii stages rows 16 ii .. 16 ii + 15,
//         lane l slot l % 4 of row r = 16 ii + l / 4, which holds the quarter (l % 4) ^
//         ((r / 2) % 4) of the row (so an MFMA operand read of 16 consecutive rows from any first
//         row meets no LDS bank conflict; bf16 tiles of a two-buffer ring), or the quarter l % 4
//         (the others); the lane's source is x, the slot's history copy (rows
//         left of position 0 when streaming, EXEC-masked per source) or nothing (causal zero
//         padding, written once as zeros into both ring buffers);
//       - weights [BCO][TAPS * 4 + 2] 16-byte slots per column (taps x 32 channels plus two pad
//         slots: a row pitch of 2 mod 4 slots, the pitch at which the 16 column rows an MFMA
//         operand read touches meet no bank conflict); pad slots reload a real piece. E4M3
//         weights keep their bytes in LDS
//         ([BCO][TAPS * 2 + 1] slots, half the LDS bytes per operand read) and are widened to
//         bf16 (exactly) as the MFMA operand is read; their per-column scale is applied in the
//         epilogue.
//   * A two-buffer ring of stages, each KC 32-channel chunks: one barrier per stage, after which
//     the next stage's DMA is issued and runs during this stage's MFMAs. k = 1 and transposed
//     (two-tap) convs take several chunks per stage so each barrier covers enough matrix work.
//   * TAPS is a compile-time constant: the tap loop unrolls and the compiler schedules the next
//     tap's operand reads under the current tap's MFMAs.
//
// Streaming history is read as the staging reads it (above) and written from LDS: the workgroups
// of column tile 0 copy the last left_pad input rows of each stream row into the slot's other
// history copy once the stage holding them has landed.
//
// The epilogue (scale, bias, residual, mix, sum_out, activation, bf16/float32 stores) is
// conv_epilogue, shared with conv_mfma_kernel, so both kernels round every output alike.
#pragma once

#include "conv_kernel.h"

namespace omni_conv {

// OCC > 0: layers of a single stage (c_in == 32 KC) take a ring of one buffer, which lets OCC
// workgroups share a CU: one's DMA and epilogue run under another's matrix work.
template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_ROWS, int TAPS, int KC, bool W8 = false,
          int OCC = 0>
struct DmaTile {
  using Base = ConvTile<WAVES_CO, WAVES_P, TCO, TP, MAX_ROWS, TAPS>;  // epilogue geometry
  static constexpr int NT = Base::NT;
  static constexpr int BCO = Base::BCO;
  static constexpr int BP = Base::BP;
  static constexpr int NW = NT / 64;
  // 16-byte slots per weight row: a tap's 32 channels take 4 (bf16) or 2 (E4M3), plus pads to a
  // pitch of 2 mod 4 slots (bf16: the pitch whose 16-row operand reads are free of LDS bank
  // conflicts) or an odd pitch (E4M3, read 8 bytes a lane)
  static constexpr int WSLOTS = TAPS * (W8 ? 2 : 4);
  static constexpr int P = W8 ? WSLOTS + 1 : WSLOTS + 2;
  static constexpr int NIW = (BCO * P + 63) / 64;  // weight DMA instructions per chunk
  static constexpr int NIX = MAX_ROWS / 16;        // input-row DMA instructions per chunk
  static constexpr int W_PIECES = (NIW + NW - 1) / NW;
  static constexpr int X_PIECES = (NIX + NW - 1) / NW;
  static constexpr int XCHUNK = MAX_ROWS * kChunk;  // elements of a chunk's input rows
  static constexpr int WCHUNK = NIW * 64 * 8;       // elements of a chunk's weights
  static constexpr int BUF = KC * (XCHUNK + WCHUNK);
  static constexpr int RING = OCC > 0 ? 1 : 2;        // ring buffers
  static constexpr int WGS_PER_CU = OCC > 0 ? OCC : 1;  // workgroups the LDS and registers are sized for
  static constexpr size_t ring_bytes = RING * (size_t)BUF * 2;
  static constexpr size_t epi_bytes = (size_t)Base::EPI_ROWS * Base::EPITCH * 4;
  static constexpr size_t coef_offset = ring_bytes > epi_bytes ? ring_bytes : epi_bytes;
  static constexpr size_t lds_bytes = coef_offset + Base::coef_bytes();
  static_assert(MAX_ROWS % 16 == 0, "input rows are staged 16 per DMA instruction");
  static_assert(X_PIECES <= 16, "two mode bits per input piece in 32 bits");
  static_assert(lds_bytes * WGS_PER_CU <= 160 * 1024,
                "the ring, epilogue and coefficients of each resident workgroup fit the CU's LDS");
};

// The two-buffer ring takes most of a CU's LDS, so one workgroup runs per CU: WAVES_CO * WAVES_P / 4
// waves per SIMD, which the register allocation may assume (OCC times that with a one-buffer
// ring, OCC workgroups per CU).
template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_ROWS, int TAPS, int KC, bool W8,
          bool SPLIT, int OCC>
__global__ void __launch_bounds__(64 * WAVES_CO * WAVES_P)
    __attribute__((amdgpu_waves_per_eu((WAVES_CO * WAVES_P * (OCC > 0 ? OCC : 1) + 3) / 4,
                                       (WAVES_CO * WAVES_P * (OCC > 0 ? OCC : 1) + 3) / 4)))
    conv_dma_kernel(const ConvParams p) {
  using Tile = DmaTile<WAVES_CO, WAVES_P, TCO, TP, MAX_ROWS, TAPS, KC, W8, OCC>;
  static_assert(!(OCC > 0 && SPLIT), "a one-stage layer has no K slices");
  constexpr int NT = Tile::NT;
  constexpr int NW = Tile::NW;
  constexpr int BCO = Tile::BCO;
  constexpr int BP = Tile::BP;
  constexpr int P = Tile::P;
  extern __shared__ __attribute__((aligned(16))) u16 lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_co = wave % WAVES_CO;
  const int wave_p = wave / WAVES_CO;

  // blockIdx -> (position tile, column tile). The hardware deals workgroups to the 8 XCDs
  // round-robin (workgroup b to XCD b % 8), each XCD with its own L2: renumbered so that XCD x
  // runs the contiguous range x of logical tiles, and with the column tile fastest in that order
  // the workgroups sharing an input tile run on one XCD, back to back, and read it from its L2.
  // With split-K the K slice is the slowest index: slice s covers chunks [s * chunks / splits,
  // (s + 1) * chunks / splits) of every tile.
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int splits = SPLIT ? p.k_splits : 1;
  const int split = SPLIT ? tile / (p.p_tiles * p.n_tiles) : 0;
  const int in_split = SPLIT ? tile - split * (p.p_tiles * p.n_tiles) : tile;
  const int n_tile = in_split % p.n_tiles;
  const int p_tile = in_split / p.n_tiles;
  const int n0 = n_tile * BCO;

  const int dil = p.dil;
  const int lpad = p.lpad;
  const int halo = p.halo;
  const int L = p.length;
  const int XL = p.x_length;
  const int H = lpad;
  const int c_in = p.c_in;
  const int n_cols = p.n_cols;
  const int chunks = c_in / kChunk / splits;  // the launcher requires c_in % (32 KC splits) == 0
  const int c_first = split * chunks;          // the slice's first chunk
  const int stages = chunks / KC;

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

  // Input-row DMA descriptors. Piece u of thread tid is LDS slot tid % 4 of row r = tid / 4 +
  // u * NT / 4 (instruction ii = wave + u * NW, lane l: row 16 ii + l / 4), which holds the row's
  // channels lq8 .. lq8 + 7, lq8 = 8 ((tid % 4) ^ ((r / 2) % 4)): its element offset at channel
  // lq8 of chunk 0 in x or in the history pool, its source (2 bits: 0 zeros, 1 x, 2 history,
  // 3 not staged) and, when it is a sample of the new history this workgroup writes, its offset
  // there.
  const int q8 = (tid & 3) * 8;  // the LDS slot's element offset in its row
  // (the swizzle's address arithmetic on each operand read costs the one-buffer-ring tiles,
  // sized for four workgroups per CU, and the 16-wave E4M3 tile spills: they keep the quarters
  // in order)
  constexpr bool kSwizzle = OCC == 0 && !W8;
  int xoff[Tile::X_PIECES];
  int hwoff[Tile::X_PIECES];
  unsigned xmode = 0;
  const bool may_write_history = p.hist != nullptr && n_tile == 0 && H > 0;
#pragma unroll
  for (int u = 0; u < Tile::X_PIECES; ++u) {
    const int r = (tid >> 2) + u * (NT / 4);
    const int lq8 = kSwizzle ? ((tid & 3) ^ ((r >> 1) & 3)) * 8 : q8;
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
        off = (int)(slot * p.hist_slot_stride + (parity * H + (H + pos)) * (int64_t)c_in) + lq8;
        mode = 2;
      }
      if (may_write_history && slot >= 0 && pos >= XL - H && pos < XL) {
        // each sample of the new history is written by the workgroup whose tile holds it (the
        // samples left of 0 by the one holding position 0)
        const int64_t m = (int64_t)b * L + pos;
        const bool owned = pos >= 0 ? (m >= m0 && m < m_end) : row_start;
        if (owned)
          hw = (int)(slot * p.hist_slot_stride + ((1 - parity) * H + (pos - (XL - H))) *
                                                     (int64_t)c_in) + lq8;
      }
    }
    xoff[u] = off;
    hwoff[u] = hw;
    xmode |= mode << (2 * u);
  }

  // Weight DMA descriptors: slot s = 64 * (wave + u * NW) + lane of a chunk's weight area is
  // column s / P, piece s % P (tap piece / 4, quarter piece % 4; piece TAPS * 4 is the pad). The
  // packed weights of a chunk's column tile are [BCO][TAPS][32] contiguous, so the byte offset
  // within the tile is (n * TAPS * 4 + piece) * 16.
  uint32_t woff[Tile::W_PIECES];
#pragma unroll
  for (int u = 0; u < Tile::W_PIECES; ++u) {
    const int s = (wave + u * NW) * 64 + lane;
    const int n = s / P;
    const int piece = s - n * P;
    woff[u] = (n < BCO && piece < Tile::WSLOTS) ? (uint32_t)(n * Tile::WSLOTS + piece) * 16 : 0u;
  }

  // A split-K slice stores its raw float32 partial tile: the epilogue without scale, bias,
  // residual or activation, into the slice's part of the partial buffer.
  ConvParams q = p;
  if constexpr (SPLIT) {
    q.wscale = nullptr;
    q.bias = nullptr;
    q.residual = nullptr;
    q.mix_a = nullptr;
    q.mix_b = nullptr;
    q.out = nullptr;
    q.act = OMNI_ACT_NONE;
    q.sum_out = p.partial + (int64_t)split * M * n_cols;
    q.r_f16 = 0;
    q.r_st = n_cols;
    q.r_sb = (int64_t)L * n_cols;
    q.r_bytes = (uint32_t)((int64_t)M * n_cols * 4);
  }
  float* coef = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(lds) + Tile::coef_offset);
  stage_coefficients<BCO, NT, false>(q, coef, n0);

  auto xs_of = [&](int buf, int c) __attribute__((always_inline)) -> u16* {
    return lds + buf * Tile::BUF + c * (Tile::XCHUNK + Tile::WCHUNK);
  };

  // Zero padding rows: written once into every chunk of the ring's buffers (no DMA writes them).
#pragma unroll
  for (int u = 0; u < Tile::X_PIECES; ++u) {
    if (((xmode >> (2 * u)) & 3u) == 0u) {
      const int r = (tid >> 2) + u * (NT / 4);
      for (int bc = 0; bc < Tile::RING * KC; ++bc)
        *reinterpret_cast<u32x4*>(xs_of(bc / KC, bc % KC) + r * kChunk + q8) = u32x4{0u, 0u, 0u, 0u};
    }
  }

  const u16* hist = p.hist;
  const auto x_rsrc = buffer_rsrc(p.x, p.x_bytes);
  const auto h_rsrc = buffer_rsrc(p.hist, p.hist_bytes);
  const auto w_rsrc = buffer_rsrc(p.weight, p.w_bytes);
  // (offsets go to the DMA builtin as int conversions of unsigned byte offsets: other forms of
  // these arguments have made this compiler omit the kernel's host-side launch stub)
  typedef __attribute__((address_space(3))) void* lds_ptr_t;

  // The DMA of stage s (chunks s * KC ..) into ring buffer s % 2.
  auto issue = [&](int s) __attribute__((always_inline)) {
    const int buf = s & 1;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int kc = c_first + s * KC + c;
      {
        u16* xs = xs_of(buf, c);
        u16* ws = xs + Tile::XCHUNK;
        const uint32_t wbase = (uint32_t)(kc * n_cols + n0) * (uint32_t)(Tile::WSLOTS * 16);
#pragma unroll
        for (int u = 0; u < Tile::W_PIECES; ++u) {
          const int iw = wave + u * NW;
          if (iw < Tile::NIW)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(ws + iw * 64 * 8), 16,
                                                     (int)woff[u], (int)wbase, 0, 0);
        }
        const uint32_t xbase = (uint32_t)(kc * kChunk * 2);
        // the rows from x, then those from the history pool, whose DMA carries the non-temporal
        // hint (aux 2): DMAs that differ only in their buffer descriptor are merged by the
        // compiler into one whose descriptor differs between lanes, a readfirstlane loop per
        // instruction
#pragma unroll
        for (int u = 0; u < Tile::X_PIECES; ++u) {
          const int ii = wave + u * NW;
          if (ii < Tile::NIX && ((xmode >> (2 * u)) & 3u) == 1u)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rsrc, (lds_ptr_t)(xs + ii * 64 * 8), 16,
                                                     (int)((uint32_t)xoff[u] * 2u), (int)xbase, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < Tile::X_PIECES; ++u) {
          const int ii = wave + u * NW;
          if (ii < Tile::NIX && ((xmode >> (2 * u)) & 3u) == 2u)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(h_rsrc, (lds_ptr_t)(xs + ii * 64 * 8), 16,
                                                     (int)((uint32_t)xoff[u] * 2u), (int)xbase, 0, 2);
        }
      }
    }
  };

  // The new history samples of stage s, from LDS to the slot's other copy.
  auto write_history = [&](int s) __attribute__((always_inline)) {
    const int buf = s & 1;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int kc = c_first + s * KC + c;
      {
        const u16* xs = xs_of(buf, c);
#pragma unroll
        for (int u = 0; u < Tile::X_PIECES; ++u) {
          if (hwoff[u] >= 0) {
            const int r = (tid >> 2) + u * (NT / 4);
            const u32x4 v = *reinterpret_cast<const u32x4*>(xs + r * kChunk + q8);
            __builtin_amdgcn_raw_buffer_store_b128(v, h_rsrc, (uint32_t)(hwoff[u] + kc * kChunk) * 2,
                                                   0, 0);
          }
        }
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

  issue(0);
  for (int s = 0; s < stages; ++s) {
    // this wave's DMA of stage s (and its history stores) have completed; the barrier makes
    // every wave's visible and retires every read of the other buffer, which stage s + 1 refills
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (s + 1 < stages) issue(s + 1);
    if (hist != nullptr) write_history(s);
    // The stage's KC x TAPS (chunk, tap) steps, software-pipelined: the operands of step i + 1
    // are read from LDS before the MFMAs of step i, so the reads hide under the matrix work.
    const u16* xs0 = xs_of(s & 1, 0);
    auto load_step = [&](int i, bf16x8 (&a)[TCO], bf16x8 (&bv)[TP]) __attribute__((always_inline)) {
      const int c = i / TAPS;
      const int j = i - c * TAPS;
      const u16* xs = xs0 + c * (Tile::XCHUNK + Tile::WCHUNK);
      if constexpr (W8) {
        // the lane's 8 weight bytes of tap j (channels lk .. lk + 7), widened to bf16 (exact)
        const u16* wtap = xs + Tile::XCHUNK + (wco0 + lrow) * P * 8 + j * (kChunk / 2) + lk / 2;
#pragma unroll
        for (int cc = 0; cc < TCO; ++cc)
          a[cc] = __builtin_bit_cast(
              bf16x8, fp8x8_to_bf16x8(*reinterpret_cast<const u32x2*>(wtap + cc * 16 * P * 8)));
      } else {
        const u16* wtap = xs + Tile::XCHUNK + (wco0 + lrow) * P * 8 + lk + j * kChunk;
#pragma unroll
        for (int cc = 0; cc < TCO; ++cc)
          a[cc] = *reinterpret_cast<const bf16x8*>(wtap + cc * 16 * P * 8);
      }
      const int shift = j * dil;
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const int row = xrow[t] + shift;  // its quarter lane / 16 in slot (lane / 16) ^ ((row / 2) % 4)
        bv[t] = *reinterpret_cast<const bf16x8*>(
            xs + row * kChunk + (kSwizzle ? ((((lane >> 4) ^ (row >> 1)) & 3) << 3) : lk));
      }
    };
    bf16x8 a[2][TCO], bv[2][TP];
    load_step(0, a[0], bv[0]);
#pragma unroll
    for (int i = 0; i < KC * TAPS; ++i) {
      if (i + 1 < KC * TAPS) load_step(i + 1, a[(i + 1) & 1], bv[(i + 1) & 1]);
#pragma unroll
      for (int t = 0; t < TP; ++t)
#pragma unroll
        for (int cc = 0; cc < TCO; ++cc)
          acc[cc][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i & 1][cc], bv[i & 1][t],
                                                               acc[cc][t], 0, 0, 0);
    }
  }

  conv_epilogue<typename Tile::Base, WAVES_P, TCO, TP>(q, acc, lds, coef, kScale, kBias, n0, m0,
                                                       m_end, wave_p, wco0);
}

template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_ROWS, int TAPS, int KC, bool W8 = false,
          bool SPLIT = false, int OCC = 0>
struct DmaConfig {
  using Tile = DmaTile<WAVES_CO, WAVES_P, TCO, TP, MAX_ROWS, TAPS, KC, W8, OCC>;

  // Staged rows of the fullest tile: BP positions over at most nseg row segments, each with its
  // own halo.
  static int64_t rows_needed(const ConvParams& p) {
    const int64_t bp = Tile::BP;
    int64_t nseg = (bp + p.length - 2) / p.length + 1;
    if (nseg > p.batch) nseg = p.batch;
    return bp + nseg * p.halo;
  }

  // The layer's taps, whole stages of input channels, the staged rows, and at most an eighth of
  // the column tiles' matrix work wasted on columns past n_cols (narrow layers take
  // conv_mfma_kernel's narrower tiles).
  static bool fits(const ConvParams& p) {
    const int64_t padded = (p.n_cols + Tile::BCO - 1) / Tile::BCO * Tile::BCO;
    return p.taps == TAPS && (p.k_splits > 1) == SPLIT &&
           p.c_in % (kChunk * KC * p.k_splits) == 0 && (OCC == 0 || p.c_in == kChunk * KC) &&
           rows_needed(p) <= MAX_ROWS &&
           (padded - p.n_cols) * 8 <= p.n_cols;
  }

  static int64_t workgroups(const ConvParams& p) {
    const int64_t positions = (int64_t)p.batch * p.length;
    return ((positions + Tile::BP - 1) / Tile::BP) * ((p.n_cols + Tile::BCO - 1) / Tile::BCO) *
           p.k_splits;
  }

  static int launch(ConvParams p, hipStream_t stream) {
    const int64_t positions = (int64_t)p.batch * p.length;
    p.p_tiles = (int)((positions + Tile::BP - 1) / Tile::BP);
    p.n_tiles = (int)((p.n_cols + Tile::BCO - 1) / Tile::BCO);
    auto k = conv_dma_kernel<WAVES_CO, WAVES_P, TCO, TP, MAX_ROWS, TAPS, KC, W8, SPLIT, OCC>;
    // raised once per instantiation, on its first launch (no attribute calls inside a capture)
    static const bool raised = raise_lds_limit((const void*)k);
    (void)raised;
    hipLaunchKernelGGL(k, dim3((unsigned)(p.p_tiles * p.n_tiles * p.k_splits)), dim3(Tile::NT),
                       Tile::lds_bytes, stream, p);
    OMNI_LAUNCH_CHECK();
    return OMNI_OK;
  }
};

// Launch the first configuration in the list that fits and gives at least one workgroup per CU
// (256); failing that, the fitting one with the most workgroups; OMNI_ERR_UNSUPPORTED when none
// fits (the caller then takes conv_mfma_kernel). The lists are ordered by measured speed on the
// decoder's layer shapes. A forced choice (Choice::force) takes the list's entry instead.
template <typename... Cfgs>
int launch_first_fit(const ConvParams& p, Choice& ch, hipStream_t stream) {
  constexpr int64_t min_wgs = 256;
  constexpr int n = sizeof...(Cfgs);
  const bool fits[n] = {Cfgs::fits(p)...};
  const int64_t wgs[n] = {Cfgs::workgroups(p)...};
  int (*const launch[n])(ConvParams, hipStream_t) = {&Cfgs::launch...};
  int pick = -1, most = -1;
  for (int i = 0; i < n; ++i) {
    if (!fits[i]) continue;
    if (pick < 0 && wgs[i] >= min_wgs) pick = i;
    if (most < 0 || wgs[i] > wgs[most]) most = i;
  }
  if (pick < 0) pick = most;
  return choose_and_launch(ch, n, fits, wgs, launch, pick, p, stream);
}

// Launchers by tap count (1: k = 1 convs, 2: transposed convs of kernel 2 * stride, 7: k = 7
// convs; 3 and 11: narrow layers' k = 3 and k = 11 convs), one translation unit each.
// `fp8`: the packed weights are E4M3 (one byte per weight, per-column scales in the epilogue).
int launch_dma_taps1(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream);
int launch_dma_taps2(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream);
int launch_dma_taps7(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream);
// HiFiGAN's layers only (bf16 weights; n_cols <= 64, or a multiple of 128 or 96 for k = 3, or 128
// for k = 11): k = 3 and k = 11
int launch_dma_taps3(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream);
int launch_dma_taps11(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream);

}  // namespace omni_conv
