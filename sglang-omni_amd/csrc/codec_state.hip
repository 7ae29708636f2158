// In-place exchanges of per-slot codec state with the reference's exact semantics, and the
// end-of-step slot advance used by the fused streaming decode.
//
// history_exchange: one thread per (row, channel) walks the history samples in increasing order.
// Sample s of the new history reads the old history at s + new_samples (> s, so not yet
// overwritten by this thread) or a new sample; the padded front gets old[s] before pool[s] is
// replaced. No two threads touch the same (slot, channel), so no barrier is needed (rows name
// distinct slots, as the reference requires).
#include "common.h"

namespace {

template <int DT>
struct Elem;
template <>
struct Elem<OMNI_DTYPE_F32> {
  using T = float;
  static __device__ float f(T v) { return v; }
  static __device__ T r(float v) { return v; }
};
template <>
struct Elem<OMNI_DTYPE_BF16> {
  using T = u16;
  static __device__ float f(T v) { return bits_to_float_bf16(v); }
  static __device__ T r(float v) { return float_to_bits_bf16(v); }
};
template <>
struct Elem<OMNI_DTYPE_F16> {
  using T = u16;
  static __device__ float f(T v) { return bits_to_float_f16(v); }
  static __device__ T r(float v) { return float_to_bits_f16(v); }
};

template <int DT>
__global__ void history_exchange_kernel(typename Elem<DT>::T* padded, int64_t rows,
                                        int64_t channels, int64_t ps_r, int64_t ps_s,
                                        int64_t ps_c, typename Elem<DT>::T* pool,
                                        int64_t num_slots, int64_t H,
                                        int64_t hs_slot, int64_t hs_s, int64_t hs_c,
                                        const int64_t* slot_index, int64_t new_samples,
                                        int64_t tail_samples, int is_cold) {
  using T = typename Elem<DT>::T;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * channels) return;
  const int64_t row = idx / channels;
  const int64_t c = idx - row * channels;
  const int64_t slot = slot_index[row];
  if (slot < 0 || slot >= num_slots) return;
  T* prow = padded + row * ps_r + c * ps_c;
  T* hrow = pool + slot * hs_slot + c * hs_c;
  const T zero = Elem<DT>::r(0.f);
  for (int64_t s = 0; s < H; ++s) {
    const T old_s = is_cold ? zero : hrow[s * hs_s];
    const int64_t src = s + new_samples;
    T next;
    if (src < H) next = is_cold ? zero : hrow[src * hs_s];
    else next = prow[src * ps_s];
    prow[s * ps_s] = old_s;
    hrow[s * hs_s] = next;
  }
  for (int64_t q = 0; q < tail_samples; ++q) prow[(H + new_samples + q) * ps_s] = zero;
}

template <int DT>
__global__ void overlap_exchange_kernel(typename Elem<DT>::T* output, int64_t rows,
                                        int64_t channels, int64_t os_r, int64_t os_s,
                                        int64_t os_c, typename Elem<DT>::T* pool,
                                        int64_t num_slots, int64_t O,
                                        int64_t hs_slot, int64_t hs_s, int64_t hs_c,
                                        const int64_t* slot_index, int64_t emitted, int is_cold) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * channels * O) return;
  const int64_t s = idx % O;
  const int64_t rc = idx / O;
  const int64_t row = rc / channels;
  const int64_t c = rc - row * channels;
  const int64_t slot = slot_index[row];
  if (slot < 0 || slot >= num_slots) return;
  auto* orow = output + row * os_r + c * os_c;
  auto* hrow = pool + slot * hs_slot + c * hs_c;
  const auto tail = orow[(emitted + s) * os_s];
  if (!is_cold) {
    const float head = Elem<DT>::f(orow[s * os_s]);
    const float prev = Elem<DT>::f(hrow[s * hs_s]);
    orow[s * os_s] = Elem<DT>::r(head + prev);
  }
  hrow[s * hs_s] = tail;
}

__global__ void advance_slots_kernel(int64_t* parity, int64_t num_slots,
                                     const int64_t* slot_index, int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int64_t slot = slot_index[r];
  if (slot >= 0 && slot < num_slots) parity[slot] += 1;
}

bool float_like(int dt) {
  return dt == OMNI_DTYPE_F32 || dt == OMNI_DTYPE_BF16 || dt == OMNI_DTYPE_F16;
}

}  // namespace

extern "C" int omni_history_exchange(void* padded, int dtype, int64_t rows, int64_t padded_samples,
                                     int64_t channels, int64_t padded_stride_row,
                                     int64_t padded_stride_sample, int64_t padded_stride_channel,
                                     void* history_pool, int64_t num_slots,
                                     int64_t history_samples, int64_t pool_stride_slot, int64_t pool_stride_sample,
                                     int64_t pool_stride_channel, const int64_t* slot_index,
                                     int64_t new_samples, int is_cold, omni_stream_t stream) {
  if (!padded || !history_pool || !slot_index || !float_like(dtype)) return OMNI_ERR_INVALID_ARG;
  if (rows < 0 || channels < 0 || history_samples < 0 || new_samples < 0)
    return OMNI_ERR_INVALID_ARG;
  const int64_t tail = padded_samples - history_samples - new_samples;
  if (tail < 0) return OMNI_ERR_INVALID_ARG;
  if (rows == 0 || channels == 0) return OMNI_OK;
  const int64_t n = rows * channels;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == OMNI_DTYPE_F32)
    hipLaunchKernelGGL(history_exchange_kernel<OMNI_DTYPE_F32>, grid, block, 0, s,
                       reinterpret_cast<float*>(padded), rows, channels, padded_stride_row,
                       padded_stride_sample, padded_stride_channel,
                       reinterpret_cast<float*>(history_pool), num_slots, history_samples, pool_stride_slot,
                       pool_stride_sample, pool_stride_channel, slot_index, new_samples, tail,
                       is_cold);
  else if (dtype == OMNI_DTYPE_BF16)
    hipLaunchKernelGGL(history_exchange_kernel<OMNI_DTYPE_BF16>, grid, block, 0, s,
                       reinterpret_cast<u16*>(padded), rows, channels, padded_stride_row,
                       padded_stride_sample, padded_stride_channel,
                       reinterpret_cast<u16*>(history_pool), num_slots, history_samples, pool_stride_slot,
                       pool_stride_sample, pool_stride_channel, slot_index, new_samples, tail,
                       is_cold);
  else
    hipLaunchKernelGGL(history_exchange_kernel<OMNI_DTYPE_F16>, grid, block, 0, s,
                       reinterpret_cast<u16*>(padded), rows, channels, padded_stride_row,
                       padded_stride_sample, padded_stride_channel,
                       reinterpret_cast<u16*>(history_pool), num_slots, history_samples, pool_stride_slot,
                       pool_stride_sample, pool_stride_channel, slot_index, new_samples, tail,
                       is_cold);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_overlap_exchange(void* output, int dtype, int64_t rows, int64_t channels,
                                     int64_t output_stride_row, int64_t output_stride_sample,
                                     int64_t output_stride_channel, void* overlap_pool,
                                     int64_t num_slots, int64_t overlap_samples, int64_t pool_stride_slot,
                                     int64_t pool_stride_sample, int64_t pool_stride_channel,
                                     const int64_t* slot_index, int64_t emitted_samples,
                                     int is_cold, omni_stream_t stream) {
  if (!output || !overlap_pool || !slot_index || !float_like(dtype)) return OMNI_ERR_INVALID_ARG;
  if (rows < 0 || channels < 0 || overlap_samples < 0) return OMNI_ERR_INVALID_ARG;
  if (emitted_samples < overlap_samples) return OMNI_ERR_INVALID_ARG;
  const int64_t n = rows * channels * overlap_samples;
  if (n == 0) return OMNI_OK;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == OMNI_DTYPE_F32)
    hipLaunchKernelGGL(overlap_exchange_kernel<OMNI_DTYPE_F32>, grid, block, 0, s,
                       reinterpret_cast<float*>(output), rows, channels, output_stride_row,
                       output_stride_sample, output_stride_channel,
                       reinterpret_cast<float*>(overlap_pool), num_slots, overlap_samples, pool_stride_slot,
                       pool_stride_sample, pool_stride_channel, slot_index, emitted_samples,
                       is_cold);
  else if (dtype == OMNI_DTYPE_BF16)
    hipLaunchKernelGGL(overlap_exchange_kernel<OMNI_DTYPE_BF16>, grid, block, 0, s,
                       reinterpret_cast<u16*>(output), rows, channels, output_stride_row,
                       output_stride_sample, output_stride_channel,
                       reinterpret_cast<u16*>(overlap_pool), num_slots, overlap_samples, pool_stride_slot,
                       pool_stride_sample, pool_stride_channel, slot_index, emitted_samples,
                       is_cold);
  else
    hipLaunchKernelGGL(overlap_exchange_kernel<OMNI_DTYPE_F16>, grid, block, 0, s,
                       reinterpret_cast<u16*>(output), rows, channels, output_stride_row,
                       output_stride_sample, output_stride_channel,
                       reinterpret_cast<u16*>(overlap_pool), num_slots, overlap_samples, pool_stride_slot,
                       pool_stride_sample, pool_stride_channel, slot_index, emitted_samples,
                       is_cold);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_advance_slots(int64_t* slot_parity, int64_t num_slots,
                                  const int64_t* slot_index, int64_t rows, omni_stream_t stream) {
  if (!slot_parity || !slot_index || rows < 0 || num_slots < 0) return OMNI_ERR_INVALID_ARG;
  if (rows == 0) return OMNI_OK;
  hipLaunchKernelGGL(advance_slots_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), slot_parity, num_slots, slot_index,
                     rows);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}
