// RVQ dequantize: gather K code-embedding rows per frame and sum them in float32.
//
// Bandwidth-bound: every frame reads K table rows of D elements, its K codes and writes one
// D-element row. One wave per frame covers D in 16-byte pieces (8 bf16 or 4 fp32 per lane per
// piece), so each table row is a fully coalesced 16-byte-per-lane load; the adds run strictly in
// k order, so float32 results are bit-identical to the sequential sum the reference computes.
//
// K <= 32 and at most 8192 frames (every codec's decode step here): rvq_gather_frame_kernel, one
// 64-thread workgroup per frame, so a decode step's few hundred frames spread over every CU. Lane k
// loads codebook k's code (one round trip for all K), the row indices are broadcast by cross-lane
// reads, and every one of the K row loads is in flight (raw 16-byte pieces held in registers)
// before the first add: a frame costs two dependent memory round trips (codes, rows) and the
// store. Larger K or batches: rvq_gather_sum_kernel, four frames per workgroup, the rows loaded
// eight at a time (many waves cover the latency there).
#include "common.h"

namespace {

constexpr int kWave = 64;
constexpr int kFramesPerBlock = 4;  // 4 waves per 256-thread block, one frame each

template <typename CodeT>
__device__ __forceinline__ int64_t load_code(const CodeT* codes, int64_t idx) {
  return (int64_t)codes[idx];
}

__device__ __forceinline__ float4 load_row4_f32(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}

// Store one lane's VEC sums at element d0 of the output row starting at element row_off: bf16
// (rounded to nearest even) or float32, 16 / 8-byte stores when the row is contiguous.
template <int VEC, bool OUT_BF16>
__device__ __forceinline__ void store_piece(const float* acc, void* __restrict__ out,
                                            int64_t row_off, int64_t d0, int64_t os_d) {
  if (OUT_BF16) {
    u16* o = reinterpret_cast<u16*>(out) + row_off;
    if (os_d == 1) {
      u16 h[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) h[e] = float_to_bits_bf16(acc[e]);
      if constexpr (VEC == 8) {
        uint4 v;
        v.x = h[0] | ((uint32_t)h[1] << 16);
        v.y = h[2] | ((uint32_t)h[3] << 16);
        v.z = h[4] | ((uint32_t)h[5] << 16);
        v.w = h[6] | ((uint32_t)h[7] << 16);
        *reinterpret_cast<uint4*>(o + d0) = v;
      } else {
        uint2 v;
        v.x = h[0] | ((uint32_t)h[1] << 16);
        v.y = h[2] | ((uint32_t)h[3] << 16);
        *reinterpret_cast<uint2*>(o + d0) = v;
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[(d0 + e) * os_d] = float_to_bits_bf16(acc[e]);
    }
  } else {
    float* o = reinterpret_cast<float*>(out) + row_off;
    if (os_d == 1 && VEC == 4) {
      *reinterpret_cast<float4*>(o + d0) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[(d0 + e) * os_d] = acc[e];
    }
  }
}

// TableT = float (4 elements / 16 B) or u16 bf16 bits (8 elements / 16 B).
template <typename CodeT, typename TableT, int VEC, bool OUT_BF16>
__global__ void __launch_bounds__(256) rvq_gather_sum_kernel(
    const CodeT* __restrict__ codes, int64_t batch, int num_codebooks, int64_t frames,
    int64_t cs_b, int64_t cs_k, int64_t cs_t, const TableT* __restrict__ table,
    int64_t codebook_size, int64_t dim, void* __restrict__ out, int64_t os_b, int64_t os_t,
    int64_t os_d, int flags) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t frame = (int64_t)blockIdx.x * kFramesPerBlock + (threadIdx.x >> 6);
  if (frame >= batch * frames) return;
  const int64_t b = frame / frames;
  const int64_t t = frame - b * frames;
  const bool clamp = (flags & OMNI_RVQ_CLAMP) != 0;

  // This lane's code (lane k holds codebook k's code; K <= 64 is checked on the host).
  // Row index into the flattened [K * V] table; K * V < 2^31 is checked on the host.
  int my_row = -1;
  if (lane < num_codebooks) {
    int64_t c = load_code(codes, b * cs_b + (int64_t)lane * cs_k + t * cs_t);
    if (c >= codebook_size && clamp) c = codebook_size - 1;
    my_row = (c >= 0 && c < codebook_size) ? (int)((int64_t)lane * codebook_size + c) : -1;
  }

  const int64_t pieces = dim / VEC;  // dim % VEC == 0 is checked on the host
  // The trip count is wave-uniform so every lane is active at the cross-lane reads below;
  // lanes past the row's end only skip their loads and stores.
  for (int64_t base = 0; base < pieces; base += kWave) {
    const int64_t piece = base + lane;
    const bool in_row = piece < pieces;
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int k0 = 0; k0 < num_codebooks; k0 += 8) {
      float vals[8][VEC];
      bool valid[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u;
        // k is wave-uniform: read lane k's row into a scalar register.
        const int row = k < num_codebooks ? __builtin_amdgcn_readlane(my_row, k) : -1;
        valid[u] = row >= 0;
        if (valid[u] && in_row) {
          const TableT* src = table + (int64_t)row * dim + piece * VEC;
          if constexpr (VEC == 4) {
            float4 v = load_row4_f32(reinterpret_cast<const float*>(src));
            vals[u][0] = v.x; vals[u][1] = v.y; vals[u][2] = v.z; vals[u][3] = v.w;
          } else {
            uint4 v = *reinterpret_cast<const uint4*>(src);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              vals[u][2 * q] = __uint_as_float(w[q] << 16);
              vals[u][2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) vals[u][e] = 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (k0 + u < num_codebooks && valid[u]) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[e] = acc[e] + vals[u][e];
        }
      }
    }
    if (flags & OMNI_RVQ_MEAN) {
      const float kf = (float)num_codebooks;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = acc[e] / kf;
    }
    if (!in_row) continue;
    store_piece<VEC, OUT_BF16>(acc, out, b * os_b + t * os_t, piece * VEC, os_d);
  }
}

// K <= KMAX codebooks, one 64-thread workgroup per frame (fewer than 2^31 frames, each with
// fewer than 2^31 elements of codes: 32-bit index arithmetic): lane k loads codebook k's code
// (one round trip for all of them), the row indices are broadcast by cross-lane reads into
// scalar registers, and the K row pieces are loaded as raw 16-byte values, all in flight before
// the first add, then widened and added in k order.
template <typename CodeT, typename TableT, int VEC, bool OUT_BF16, int KMAX>
__global__ void __launch_bounds__(64) rvq_gather_frame_kernel(
    const CodeT* __restrict__ codes, int num_codebooks, int frames, int64_t cs_b, int64_t cs_k,
    int64_t cs_t, const TableT* __restrict__ table, int codebook_size, int dim,
    void* __restrict__ out, int64_t os_b, int64_t os_t, int64_t os_d, int flags) {
  const int lane = threadIdx.x;
  const int frame = blockIdx.x;
  const int b = frame / frames;
  const int t = frame - b * frames;
  const bool clamp = (flags & OMNI_RVQ_CLAMP) != 0;
  // Row index of the lane's codebook's code into the flattened [K * V] table (-1: the code adds
  // nothing); K * V < 2^31 is checked on the host.
  int my_row = -1;
  if (lane < num_codebooks) {
    int64_t c = (int64_t)codes[b * cs_b + (int64_t)lane * cs_k + t * cs_t];
    if (c >= codebook_size && clamp) c = codebook_size - 1;
    my_row = (c >= 0 && c < codebook_size) ? lane * codebook_size + (int)c : -1;
  }
  int rows[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) rows[k] = __builtin_amdgcn_readlane(my_row, k);
  const int pieces = dim / VEC;  // dim % VEC == 0 is checked on the host
  for (int piece = lane; piece < pieces; piece += kWave) {
    uint4 raw[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      raw[k] = uint4{0u, 0u, 0u, 0u};
      if (rows[k] >= 0)
        raw[k] = *reinterpret_cast<const uint4*>(table + (int64_t)rows[k] * dim + piece * VEC);
    }
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if (rows[k] < 0) continue;
      const uint32_t w[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
      if constexpr (VEC == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = acc[e] + __uint_as_float(w[e]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = acc[2 * q] + __uint_as_float(w[q] << 16);
          acc[2 * q + 1] = acc[2 * q + 1] + __uint_as_float(w[q] & 0xffff0000u);
        }
      }
    }
    if (flags & OMNI_RVQ_MEAN) {
      const float kf = (float)num_codebooks;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = acc[e] / kf;
    }
    store_piece<VEC, OUT_BF16>(acc, out, b * os_b + t * os_t, (int64_t)piece * VEC, os_d);
  }
}

template <typename CodeT, typename TableT, int VEC, bool OUT_BF16>
void launch_frames(const CodeT* c, int64_t batch, int k, int64_t frames, int64_t cs_b,
                   int64_t cs_k, int64_t cs_t, const TableT* t, int64_t v, int64_t dim, void* out,
                   int64_t os_b, int64_t os_t, int64_t os_d, int flags, hipStream_t stream) {
  const dim3 grid((unsigned)(batch * frames)), block(64);
  const int fr = (int)frames, vi = (int)v, di = (int)dim;
  if (k <= 8)
    hipLaunchKernelGGL((rvq_gather_frame_kernel<CodeT, TableT, VEC, OUT_BF16, 8>), grid, block, 0,
                       stream, c, k, fr, cs_b, cs_k, cs_t, t, vi, di, out, os_b, os_t, os_d, flags);
  else if (k <= 16)
    hipLaunchKernelGGL((rvq_gather_frame_kernel<CodeT, TableT, VEC, OUT_BF16, 16>), grid, block,
                       0, stream, c, k, fr, cs_b, cs_k, cs_t, t, vi, di, out, os_b, os_t, os_d,
                       flags);
  else
    hipLaunchKernelGGL((rvq_gather_frame_kernel<CodeT, TableT, VEC, OUT_BF16, 32>), grid, block,
                       0, stream, c, k, fr, cs_b, cs_k, cs_t, t, vi, di, out, os_b, os_t, os_d,
                       flags);
}

// The frame kernel takes decode-step sizes (latency-bound: a few thousand frames or fewer);
// large batches keep the four-frame workgroups, whose many waves already cover the latency
// (12 000 frames of 32 codebooks: 51.5 against 53.8 us).
constexpr int kFrameKernelMaxK = 32;
constexpr int64_t kFrameKernelMaxFrames = 8192;

template <typename CodeT>
int launch_rvq(const void* codes, int64_t batch, int64_t k, int64_t frames, int64_t cs_b,
               int64_t cs_k, int64_t cs_t, const void* table, int table_dtype, int64_t v,
               int64_t dim, void* out, int out_dtype, int64_t os_b, int64_t os_t, int64_t os_d,
               int flags, hipStream_t stream) {
  const int64_t total = batch * frames;
  const dim3 grid((unsigned)((total + kFramesPerBlock - 1) / kFramesPerBlock));
  const dim3 block(256);
  const CodeT* c = reinterpret_cast<const CodeT*>(codes);
  const bool out_bf16 = out_dtype == OMNI_DTYPE_BF16;
  if (k <= kFrameKernelMaxK && total <= kFrameKernelMaxFrames && dim <= 0x7fffffff) {
    if (table_dtype == OMNI_DTYPE_F32) {
      const float* t = reinterpret_cast<const float*>(table);
      if (out_bf16)
        launch_frames<CodeT, float, 4, true>(c, batch, (int)k, frames, cs_b, cs_k, cs_t, t, v,
                                             dim, out, os_b, os_t, os_d, flags, stream);
      else
        launch_frames<CodeT, float, 4, false>(c, batch, (int)k, frames, cs_b, cs_k, cs_t, t, v,
                                              dim, out, os_b, os_t, os_d, flags, stream);
    } else {
      const u16* t = reinterpret_cast<const u16*>(table);
      if (out_bf16)
        launch_frames<CodeT, u16, 8, true>(c, batch, (int)k, frames, cs_b, cs_k, cs_t, t, v, dim,
                                           out, os_b, os_t, os_d, flags, stream);
      else
        launch_frames<CodeT, u16, 8, false>(c, batch, (int)k, frames, cs_b, cs_k, cs_t, t, v,
                                            dim, out, os_b, os_t, os_d, flags, stream);
    }
    OMNI_LAUNCH_CHECK();
    return OMNI_OK;
  }
  if (table_dtype == OMNI_DTYPE_F32) {
    const float* t = reinterpret_cast<const float*>(table);
    if (out_bf16)
      hipLaunchKernelGGL((rvq_gather_sum_kernel<CodeT, float, 4, true>), grid, block, 0, stream,
                         c, batch, (int)k, frames, cs_b, cs_k, cs_t, t, v, dim, out, os_b, os_t,
                         os_d, flags);
    else
      hipLaunchKernelGGL((rvq_gather_sum_kernel<CodeT, float, 4, false>), grid, block, 0, stream,
                         c, batch, (int)k, frames, cs_b, cs_k, cs_t, t, v, dim, out, os_b, os_t,
                         os_d, flags);
  } else {
    const u16* t = reinterpret_cast<const u16*>(table);
    if (out_bf16)
      hipLaunchKernelGGL((rvq_gather_sum_kernel<CodeT, u16, 8, true>), grid, block, 0, stream, c,
                         batch, (int)k, frames, cs_b, cs_k, cs_t, t, v, dim, out, os_b, os_t,
                         os_d, flags);
    else
      hipLaunchKernelGGL((rvq_gather_sum_kernel<CodeT, u16, 8, false>), grid, block, 0, stream,
                         c, batch, (int)k, frames, cs_b, cs_k, cs_t, t, v, dim, out, os_b, os_t,
                         os_d, flags);
  }
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

}  // namespace

extern "C" int omni_rvq_gather_sum(const void* codes, int codes_dtype, int64_t batch,
                                   int64_t num_codebooks, int64_t frames, int64_t codes_stride_b,
                                   int64_t codes_stride_k, int64_t codes_stride_t,
                                   const void* codebooks, int table_dtype, int64_t codebook_size,
                                   int64_t dim, void* out, int out_dtype, int64_t out_stride_b,
                                   int64_t out_stride_t, int64_t out_stride_d, int flags,
                                   omni_stream_t stream) {
  if (!codes || !codebooks || !out) return OMNI_ERR_INVALID_ARG;
  if (batch < 0 || frames < 0 || num_codebooks < 1 || num_codebooks > 64 || codebook_size < 1 ||
      dim < 1)
    return OMNI_ERR_INVALID_ARG;
  if (codes_dtype != OMNI_DTYPE_I32 && codes_dtype != OMNI_DTYPE_I64) return OMNI_ERR_INVALID_ARG;
  if (table_dtype != OMNI_DTYPE_F32 && table_dtype != OMNI_DTYPE_BF16) return OMNI_ERR_INVALID_ARG;
  if (out_dtype != OMNI_DTYPE_F32 && out_dtype != OMNI_DTYPE_BF16) return OMNI_ERR_INVALID_ARG;
  if (flags & ~(OMNI_RVQ_MEAN | OMNI_RVQ_CLAMP)) return OMNI_ERR_INVALID_ARG;
  const int vec = table_dtype == OMNI_DTYPE_F32 ? 4 : 8;
  if (dim % vec) return OMNI_ERR_UNSUPPORTED;
  if (num_codebooks * codebook_size >= 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  const uintptr_t table_addr = reinterpret_cast<uintptr_t>(codebooks);
  if (table_addr % 16) return OMNI_ERR_INVALID_ARG;
  if (out_stride_d == 1) {
    const int out_bytes = out_dtype == OMNI_DTYPE_F32 ? 4 : 2;
    const int need = vec * out_bytes >= 16 ? 16 : vec * out_bytes;
    if ((reinterpret_cast<uintptr_t>(out) % need) || ((out_stride_b * out_bytes) % need) ||
        ((out_stride_t * out_bytes) % need))
      return OMNI_ERR_INVALID_ARG;
  }
  if (batch == 0 || frames == 0) return OMNI_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (codes_dtype == OMNI_DTYPE_I32)
    return launch_rvq<int32_t>(codes, batch, num_codebooks, frames, codes_stride_b,
                               codes_stride_k, codes_stride_t, codebooks, table_dtype,
                               codebook_size, dim, out, out_dtype, out_stride_b, out_stride_t,
                               out_stride_d, flags, s);
  return launch_rvq<int64_t>(codes, batch, num_codebooks, frames, codes_stride_b, codes_stride_k,
                             codes_stride_t, codebooks, table_dtype, codebook_size, dim, out,
                             out_dtype, out_stride_b, out_stride_t, out_stride_d, flags, s);
}
