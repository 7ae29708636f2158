// A HiFiGAN ResBlock pair of the 32-channel stage in one launch (gfx950 bf16 MFMA):
//
//   h = act1(c1(x))                    c1: k taps, dilation d, "same" zero padding
//   y = c2(h) (+ residual, mix, ...)   c2: k taps, dilation 1; the conv epilogue of omni_conv1d
//
// (ResBlock of sglang_omni/models/minicpm_o/components/token2wav/hift_layers.py:95-110, as
// hift.py:255-281 runs it: xt = act(x); xt = c1(xt); xt = act(xt); xt = c2(xt); x = xt + x.)
// Run as two launches, h goes to HBM as bf16 and comes back (4 bytes per element); here a
// workgroup computes h for its output positions and the c2 halo into LDS and c2 reads it there.
//
// Workgroup: 4 waves over 32 columns x BP = 64 TP output positions of one row. The x rows of the
// tile's positions and both convs' halos (r1 = (k-1) d / 2 and r2 = (k-1) / 2 on each side) and
// both weight sets are staged in LDS once (64-byte rows, slot s of row r at s ^ ((r/2) % 4), and
// weight rows of k*4 + 2 16-byte slots: the layouts whose MFMA operand reads meet no bank
// conflict); h rows outside [0, length) are zeros (c2's padding). Each accumulator takes its MFMAs
// in the order of the LDS-DMA conv kernel's (taps ascending), h rounds the way that kernel's
// epilogue rounds its bf16 output, and c2's accumulators go through the same conv_epilogue: the
// pair gives the bits of the two launches.
#include "conv_kernel.h"
#include "omni_codec.h"

namespace omni_conv {
int make_conv_params(const omni_conv_args* a, ConvParams& p, bool& x_f32, bool& fp8, bool& fuse2);
}

namespace {

using namespace omni_conv;

constexpr int kC = 32;      // channels: one 32-channel chunk
constexpr int kMaxDil = 5;  // the largest c1 dilation the LDS is sized for

template <int K, int TP>
struct PairTile {
  using Base = ConvTile<1, 4, 2, TP, 64, K>;  // the epilogue's geometry: 32 columns, 4 waves
  static constexpr int NT = Base::NT;
  static constexpr int BP = Base::BP;
  static constexpr int R2 = (K - 1) / 2;
  static constexpr int HGROUPS = (BP + 2 * R2 + 15) / 16;  // 16-row groups of h
  static constexpr int HROWS = HGROUPS * 16;
  // staged x rows: every row an h row's taps read, up to the largest dilation (rows past the
  // tile's span BP + 2 (r1 + r2) hold zeros)
  static constexpr int XROWS = (HROWS + (K - 1) * kMaxDil + 15) / 16 * 16;
  static constexpr int WP = K * 4 + 2;  // 16-byte slots per weight row
  static constexpr size_t x_bytes = (size_t)XROWS * kC * 2;
  static constexpr size_t epi_bytes = (size_t)Base::EPI_ROWS * Base::EPITCH * 4;
  static constexpr size_t h_offset = x_bytes > epi_bytes ? x_bytes : epi_bytes;
  static constexpr size_t w1_offset = h_offset + (size_t)HROWS * kC * 2;
  static constexpr size_t w2_offset = w1_offset + (size_t)kC * WP * 16;
  static constexpr size_t coef_offset = w2_offset + (size_t)kC * WP * 16;
  static constexpr size_t lds_bytes = coef_offset + Base::coef_bytes() + kC * 4;
  static_assert(lds_bytes <= 160 * 1024, "the pair's tiles fit the CU's LDS");
};

// element offset of 16-byte slot `slot` of 64-byte row `row`
__device__ __forceinline__ int row_slot(int row, int slot) {
  return row * kC + ((slot ^ ((row >> 1) & 3)) << 3);
}

template <int K, int TP>
// (three workgroups per CU where the LDS allows, k = 3; two otherwise)
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(K == 3 ? 3 : 2,
                                                                          K == 3 ? 3 : 2)))
    resblock_pair_kernel(const ConvParams c1, const ConvParams c2, int tiles_per_row) {
  using T = PairTile<K, TP>;
  constexpr int NT = T::NT;
  constexpr int BP = T::BP;
  constexpr int R2 = T::R2;
  constexpr int WP = T::WP;
  extern __shared__ __attribute__((aligned(16))) u16 lds[];
  u16* xs = lds;
  u16* hs = lds + T::h_offset / 2;
  u16* w1s = lds + T::w1_offset / 2;
  u16* w2s = lds + T::w2_offset / 2;
  float* coef = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(lds) + T::coef_offset);
  float* bias1 = coef + ConvTile<1, 4, 2, TP, 64, K>::NCOEF * kC;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 15;
  const int q = lane >> 4;
  const int L = c2.length;
  const int d = c1.dil;
  const int r1 = c1.lpad;  // (K - 1) d / 2
  const int R = r1 + R2;

  // ---- once per workgroup: both weight sets (row n: tap j's quarter s in slot 4 j + s) and the
  // coefficients, then the workgroup's tiles one after another (a grid of about one workgroup per
  // resident slot, so the weights are staged once per workgroup, not once per tile)
  {
    const auto w1r = buffer_rsrc(c1.weight, (uint32_t)(kC * K * kC * 2));
    const auto w2r = buffer_rsrc(c2.weight, (uint32_t)(kC * K * kC * 2));
    for (int e = tid; e < kC * K * 4; e += NT) {
      const int n = e / (K * 4);
      const int s = e - n * (K * 4);
      const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(w1r, (uint32_t)e * 16u, 0, 0);
      const u32x4 v2 = __builtin_amdgcn_raw_buffer_load_b128(w2r, (uint32_t)e * 16u, 0, 0);
      *reinterpret_cast<u32x4*>(w1s + (n * WP + s) * 8) = v1;
      *reinterpret_cast<u32x4*>(w2s + (n * WP + s) * 8) = v2;
    }
    stage_coefficients<kC, NT, false>(c2, coef, 0);
    for (int n = tid; n < kC; n += NT) bias1[n] = c1.bias ? c1.bias[n] : 0.f;
  }
  const auto xr = buffer_rsrc(c1.x, c1.x_bytes);
  const int tiles = tiles_per_row * c2.batch;
  // The x rows of a tile (position i0 - R + r, zeros outside [0, x_length)) go through
  // registers: with PREFETCH the next tile's are loaded as soon as this tile's are in LDS, so
  // their latency hides under this tile's convs and epilogue (k = 7, two workgroups per CU: 338-
  // 392 -> 298-348 us per pair launch at 16 x 240 000 samples); k = 3 keeps three workgroups per
  // CU, whose registers the prefetch would spill (211-259 -> 236-287 us), and loads them at the
  // tile's start.
  constexpr bool PREFETCH = K != 3;
  constexpr int XP = (T::XROWS * 4 + NT - 1) / NT;  // 16-byte pieces per thread
  u32x4 xpre[XP];
  auto load_x = [&](int t) __attribute__((always_inline)) {
    const int tb = t / tiles_per_row;
    const int ti0 = (t - tb * tiles_per_row) * BP;
    const int rows = BP + 2 * R;  // staged rows the tile reads
#pragma unroll
    for (int u = 0; u < XP; ++u) {
      const int e = tid + u * NT;
      const int r = e >> 2;
      const int pos = ti0 - R + r;
      const bool ok = e < T::XROWS * 4 && r < rows && pos >= 0 && pos < c1.x_length;
      const uint32_t off = ok ? (uint32_t)((int64_t)tb * c1.x_sb + (int64_t)pos * c1.x_st +
                                           (e & 3) * 8) * 2u
                              : kOutOfRange;
      xpre[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
    }
  };
  if (PREFETCH && (int)blockIdx.x < tiles) load_x(blockIdx.x);
  for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
  const int b = tile / tiles_per_row;
  const int i0 = (tile - b * tiles_per_row) * BP;
  const int m0 = b * L + i0;
  const int m_end = m0 + min(BP, L - i0);

  // ---- the tile's x rows into LDS, once the previous tile's epilogue has read its rows of the
  // (aliased) x area; then the next tile's loads
  if (!PREFETCH) load_x(tile);
  __syncthreads();
#pragma unroll
  for (int u = 0; u < XP; ++u) {
    const int e = tid + u * NT;
    if (e < T::XROWS * 4) *reinterpret_cast<u32x4*>(xs + row_slot(e >> 2, e & 3)) = xpre[u];
  }
  if (PREFETCH && tile + (int)gridDim.x < tiles) load_x(tile + gridDim.x);
  __syncthreads();

  // ---- c1 over the h rows: h row hr is position i0 - R2 + hr and reads x rows hr + j d
  {
    const u16* w1row = w1s + lrow * WP * 8 + q * 8;
    for (int g = wave; g < T::HGROUPS; g += NT / 64) {
      const int hr = g * 16 + lrow;
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int xrow = hr + j * d;
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(xs + row_slot(xrow, q));
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const bf16x8 av = *reinterpret_cast<const bf16x8*>(w1row + c * 16 * WP * 8 + j * 32);
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[c], 0, 0, 0);
        }
      }
      // the LDS-DMA conv epilogue's expression: acc * scale (1 for bf16 weights) + bias, then the
      // activation, rounded to bf16; zeros outside [0, length) (c2's padding)
      const int pos = i0 - R2 + hr;
      const bool inside = pos >= 0 && pos < L;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int n = c * 16 + q * 4;
        const f32x4 sc = *reinterpret_cast<const f32x4*>(coef + kScale * kC + n);
        const f32x4 bi = *reinterpret_cast<const f32x4*>(bias1 + n);
        f32x4 v = acc[c] * sc + bi;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          y[e] = c1.act == OMNI_ACT_LEAKY_RELU ? (v[e] >= 0.f ? v[e] : v[e] * c1.slope) : v[e];
          if (!inside) y[e] = 0.f;
        }
        uint2 o;
        o.x = pack_bf16x2(y[0], y[1]);
        o.y = pack_bf16x2(y[2], y[3]);
        // channels n .. n + 3: slot n / 8 of the row, half (n / 4) % 2
        *reinterpret_cast<uint2*>(hs + row_slot(hr, n >> 3) + (n & 7)) = o;
      }
    }
  }
  __syncthreads();

  // ---- c2 over the tile's positions: output row o reads h rows o + j
  f32x4 acc[2][TP];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int t = 0; t < TP; ++t) acc[c][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    const u16* w2row = w2s + lrow * WP * 8 + q * 8;
    const int o0 = wave * TP * 16 + lrow;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      bf16x8 av[2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
        av[c] = *reinterpret_cast<const bf16x8*>(w2row + c * 16 * WP * 8 + j * 32);
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(hs + row_slot(o0 + t * 16 + j, q));
#pragma unroll
        for (int c = 0; c < 2; ++c)
          acc[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[c], bv, acc[c][t], 0, 0, 0);
      }
    }
  }
  // (the epilogue's first pass begins with a barrier; its rows overwrite only the x tile)
  conv_epilogue<typename T::Base, 4, 2, TP>(c2, acc, lds, coef, kScale, kBias, 0, m0, m_end, wave,
                                            0);
  }  // tiles
}

template <int K, int TP>
int launch(const ConvParams& p1, const ConvParams& p2, hipStream_t stream) {
  using T = PairTile<K, TP>;
  const int64_t tiles_per_row = (p2.length + T::BP - 1) / T::BP;
  const int64_t grid = tiles_per_row * p2.batch;
  if (grid > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  auto k = resblock_pair_kernel<K, TP>;
  static const bool raised = hipFuncSetAttribute((const void*)k,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)T::lds_bytes) == hipSuccess;
  if (!raised) return OMNI_ERR_LAUNCH;
  // one workgroup per resident slot of the device (LDS and registers allow `per_cu` per CU)
  static const int64_t slots = [&] {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, T::NT, T::lds_bytes) !=
            hipSuccess ||
        cus <= 0 || per_cu <= 0)
      return (int64_t)256;
    return (int64_t)cus * per_cu;
  }();
  const int64_t workgroups = grid < slots ? grid : slots;
  hipLaunchKernelGGL(k, dim3((unsigned)workgroups), dim3(T::NT), T::lds_bytes, stream, p1, p2,
                     (int)tiles_per_row);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

}  // namespace

extern "C" int omni_resblock_pair(const omni_conv_args* c1, const omni_conv_args* c2,
                                  omni_stream_t stream) {
  if (!c1 || !c2) return OMNI_ERR_INVALID_ARG;
  // c1 writes no tensor (h stays on chip) and c2 reads none (its operand is h): validate each as
  // a conv with c1's operand standing in
  if (c1->out || c1->sum_out || c1->residual || c1->mix_a || c2->x) return OMNI_ERR_INVALID_ARG;
  omni_conv_args a1 = *c1, a2 = *c2;
  a1.out = const_cast<void*>(c1->x);
  a1.out_dtype = OMNI_DTYPE_BF16;
  a1.out_stride_b = c1->x_stride_b;
  a1.out_stride_t = c1->x_stride_t;
  a2.x = c1->x;
  a2.x_dtype = c1->x_dtype;
  a2.x_stride_b = c1->x_stride_b;
  a2.x_stride_t = c1->x_stride_t;
  a2.x_length = 0;
  ConvParams p1, p2;
  bool f32a, fp8a, fuse2a, f32b, fp8b, fuse2b;
  int st = make_conv_params(&a1, p1, f32a, fp8a, fuse2a);
  if (st > 0) return st;
  const int st2 = make_conv_params(&a2, p2, f32b, fp8b, fuse2b);
  if (st2 > 0) return st2;
  // the shapes the kernel takes: 32 channels, bf16 operand and weights, k = 3 / 7 / 11 with
  // "same" padding, c1 dilation <= 5, c2 dilation 1, no input activation, history or fused conv
  const int64_t k = c1->taps;
  if (c1->c_in != kC || c1->n_cols != kC || c1->c_out != kC || c2->c_in != kC ||
      c2->n_cols != kC || c2->c_out != kC || c2->taps != k || c2->dilation != 1 ||
      (k != 3 && k != 7 && k != 11) || c1->dilation > kMaxDil ||
      c1->left_pad != (k - 1) * c1->dilation / 2 || c2->left_pad != (k - 1) / 2 ||
      f32a || fp8a || fp8b || fuse2a || fuse2b || c1->in_activation != OMNI_ACTIVATION_NONE ||
      c2->in_activation != OMNI_ACTIVATION_NONE || c1->hist_pool || c2->hist_pool ||
      (c1->activation != OMNI_ACTIVATION_NONE && c1->activation != OMNI_ACTIVATION_LEAKY_RELU) ||
      c1->batch != c2->batch || c1->length != c2->length ||
      (c1->x_length != 0 && c1->x_length != c1->length))
    return OMNI_ERR_UNSUPPORTED;
  if (st < 0 || st2 < 0) return OMNI_OK;  // nothing to do
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (k) {
    case 3: return launch<3, 4>(p1, p2, s);
    case 7: return launch<7, 4>(p1, p2, s);
    default: return launch<11, 2>(p1, p2, s);
  }
}
