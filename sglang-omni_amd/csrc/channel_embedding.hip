// The MOSS-TTS multi-channel embedding sum: out[row, :] = sum over channels c, in channel order,
// of tables[c][token_ids[row, c], :], the running total rounded to the output dtype after every
// add (the eager ordered sum's bits), ids outside [0, vocab_sizes[c]) adding nothing
// (moss_tts/channel_embedding.py:13-50).
//
// One thread owns 8 consecutive columns of a row (one 16-byte load per channel for bf16 / f16,
// two for float32, when the widths and addresses allow; element loads otherwise). Tables are
// separate allocations, reached through a device array of their addresses, with their own
// vocabulary sizes.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kCols = 8;  // columns per thread

struct ChannelEmbeddingParams {
  const void* ids;
  int ids_dtype;  // OMNI_DTYPE_I32 or OMNI_DTYPE_I64
  int64_t id_stride_row, id_stride_channel;
  int channels;
  const uint64_t* tables;  // [channels] device addresses of [vocab_c][hidden] tables
  const int64_t* vocab_sizes;
  int64_t hidden;
  void* out;  // [rows][hidden]
  int64_t col_blocks;  // workgroups per row
  int out_aligned;  // out is 16-byte aligned
};

template <int DT>
OMNI_DEVICE float round_to(float v) {
  if constexpr (DT == OMNI_DTYPE_BF16) return bits_to_float_bf16(float_to_bits_bf16(v));
  else if constexpr (DT == OMNI_DTYPE_F16) return bits_to_float_f16(float_to_bits_f16(v));
  else return v;
}

template <int DT>
OMNI_DEVICE void load8(const void* table, int64_t off, float v[kCols]) {
  if constexpr (DT == OMNI_DTYPE_F32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(table) + off);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(table) + off + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const u16*>(table) + off);
    const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u16 lo = (u16)(q[i] & 0xffff), hi = (u16)(q[i] >> 16);
      if constexpr (DT == OMNI_DTYPE_BF16) {
        v[2 * i] = bits_to_float_bf16(lo);
        v[2 * i + 1] = bits_to_float_bf16(hi);
      } else {
        v[2 * i] = bits_to_float_f16(lo);
        v[2 * i + 1] = bits_to_float_f16(hi);
      }
    }
  }
}

template <int DT>
OMNI_DEVICE void store8(void* out, int64_t off, const float v[kCols]) {
  if constexpr (DT == OMNI_DTYPE_F32) {
    float* o = static_cast<float*>(out) + off;
    *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u16 lo, hi;
      if constexpr (DT == OMNI_DTYPE_BF16) {
        lo = float_to_bits_bf16(v[2 * i]);
        hi = float_to_bits_bf16(v[2 * i + 1]);
      } else {
        lo = float_to_bits_f16(v[2 * i]);
        hi = float_to_bits_f16(v[2 * i + 1]);
      }
      q[i] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *reinterpret_cast<uint4*>(static_cast<u16*>(out) + off) = make_uint4(q[0], q[1], q[2], q[3]);
  }
}

template <int DT>
OMNI_DEVICE float load1(const void* table, int64_t off) {
  if constexpr (DT == OMNI_DTYPE_F32) return static_cast<const float*>(table)[off];
  else if constexpr (DT == OMNI_DTYPE_BF16) return bits_to_float_bf16(static_cast<const u16*>(table)[off]);
  else return bits_to_float_f16(static_cast<const u16*>(table)[off]);
}

template <int DT>
OMNI_DEVICE void store1(void* out, int64_t off, float v) {
  if constexpr (DT == OMNI_DTYPE_F32) static_cast<float*>(out)[off] = v;
  else if constexpr (DT == OMNI_DTYPE_BF16) static_cast<u16*>(out)[off] = float_to_bits_bf16(v);
  else static_cast<u16*>(out)[off] = float_to_bits_f16(v);
}

// A workgroup owns one row's columns [blockIdx % col_blocks * threads * 8, +threads * 8). Each
// wave takes the row's channels 64 at a time: lane l reads channel c0 + l's id, vocabulary size
// and table address (independent loads, all in flight) and forms its element offset (-1 when the
// id is out of range); the wave then broadcasts them channel by channel with readlane (the
// channel index is wave-uniform, so offsets and addresses are scalars) and issues the 16-byte
// gathers of GROUP channels before adding them in channel order: a row costs a few memory round
// trips instead of one dependent chain per channel, and no wave waits on another.
// A thread's 8 columns are whole when hidden % 8 == 0; the 16-byte forms are taken when the
// table or the output is also 16-byte aligned, element loads otherwise.
OMNI_DEVICE int64_t readlane64(int64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)(uint64_t)v, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <int DT, int GROUP>
__global__ __launch_bounds__(kThreads) void channel_embedding_sum_kernel(ChannelEmbeddingParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x / p.col_blocks;
  const int64_t col = ((blockIdx.x - row * p.col_blocks) * blockDim.x + threadIdx.x) * kCols;
  // a wave whose every lane is past the row's end has nothing to do; the others keep all lanes
  // for the metadata loads
  const int64_t wave_col = ((blockIdx.x - row * p.col_blocks) * blockDim.x + (threadIdx.x & ~63)) * kCols;
  if (wave_col >= p.hidden) return;
  const bool active = col < p.hidden;
  const bool whole = (p.hidden % kCols) == 0;
  const int n = !active ? 0 : p.hidden - col < kCols ? (int)(p.hidden - col) : kCols;
  float total[kCols];
#pragma unroll
  for (int i = 0; i < kCols; ++i) total[i] = 0.f;
  for (int c0 = 0; c0 < p.channels; c0 += 64) {
    const int nc = p.channels - c0 < 64 ? p.channels - c0 : 64;
    int64_t my_offset = -1, my_table = 0;
    if (lane < nc) {
      const int c = c0 + lane;
      const int64_t id_off = row * p.id_stride_row + (int64_t)c * p.id_stride_channel;
      const int64_t id = p.ids_dtype == OMNI_DTYPE_I64 ? static_cast<const int64_t*>(p.ids)[id_off]
                                                       : static_cast<const int32_t*>(p.ids)[id_off];
      my_table = (int64_t)p.tables[c];
      my_offset = (id >= 0 && id < p.vocab_sizes[c]) ? id * p.hidden : -1;
    }
    // whole 8-column pieces and every table of the block 16-byte aligned (one wave-wide test):
    // each gather a buffer load over its table row, an absent id or a lane past the row's end
    // reading zeros, so a group's loads are all issued before the first add (under a branch per
    // gather each one was waited on in turn)
    constexpr int ES = DT == OMNI_DTYPE_F32 ? 4 : 2;
    // (decode batches' 16-channel groups only: with 2 in flight the large batches ran 2.5 % slower)
    const bool fast = GROUP >= 16 && whole && p.hidden * ES < 0x7fffffffLL &&
                      __builtin_amdgcn_ballot_w64(lane < nc && (my_table & 15) != 0) == 0;
    for (int g = 0; g < nc; g += GROUP) {
      float v[GROUP][kCols];
      if (fast) {
#pragma unroll
        for (int j = 0; j < GROUP; ++j) {
          // lane reads at a clamped index and a select (a branch here would split the loads)
          const int jl = g + j < 64 ? g + j : 63;
          int64_t off = readlane64(my_offset, jl);
          off = g + j < nc ? off : -1;
          const uint64_t table = (uint64_t)readlane64(my_table, jl);
          const auto rs = buffer_rsrc(reinterpret_cast<const char*>(table) + (off >= 0 ? off : 0) * ES,
                                      off >= 0 ? (uint32_t)(p.hidden * ES) : 0u);
          const uint32_t o = active ? (uint32_t)(col * ES) : kOutOfRange;
          if constexpr (DT == OMNI_DTYPE_F32) {
            const f32x4 a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0));
            const f32x4 b = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, active ? o + 16u : kOutOfRange, 0, 0));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              v[j][i] = a[i];
              v[j][4 + i] = b[i];
            }
          } else {
            const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const u16 lo = (u16)(w[i] & 0xffff), hi = (u16)(w[i] >> 16);
              v[j][2 * i] = DT == OMNI_DTYPE_BF16 ? bits_to_float_bf16(lo) : bits_to_float_f16(lo);
              v[j][2 * i + 1] = DT == OMNI_DTYPE_BF16 ? bits_to_float_bf16(hi) : bits_to_float_f16(hi);
            }
          }
        }
      } else {
#pragma unroll
      for (int j = 0; j < GROUP; ++j) {
#pragma unroll
        for (int i = 0; i < kCols; ++i) v[j][i] = 0.f;
        const int64_t off = g + j < nc ? readlane64(my_offset, g + j) : -1;
        if (off >= 0 && active) {
          const uint64_t table = (uint64_t)readlane64(my_table, g + j);
          if (whole && (table & 15) == 0) {
            load8<DT>(reinterpret_cast<const void*>(table), off + col, v[j]);
          } else {
#pragma unroll
            for (int i = 0; i < kCols; ++i)
              if (i < n) v[j][i] = load1<DT>(reinterpret_cast<const void*>(table), off + col + i);
          }
        }
      }
      }
      // ordered adds; an out-of-range id adds 0 (which still turns a -0 total into +0)
#pragma unroll
      for (int j = 0; j < GROUP; ++j) {
        if (g + j < nc) {
#pragma unroll
          for (int i = 0; i < kCols; ++i) total[i] = round_to<DT>(total[i] + v[j][i]);
        }
      }
    }
  }
  if (!active) return;
  if (whole && p.out_aligned) {
    store8<DT>(p.out, row * p.hidden + col, total);
  } else {
#pragma unroll
    for (int i = 0; i < kCols; ++i)
      if (i < n) store1<DT>(p.out, row * p.hidden + col + i, total[i]);
  }
}

// Decode batches (64-thread workgroups): 16 channels' gathers in flight, since a few hundred
// waves cannot hide a round trip per channel. Large batches: 2, which keeps ~30 VGPRs and every
// wave on the same few tables at a time (the tables of a row's channels are re-read by other rows
// from cache); 8 in flight ran 12 % slower at 4096 rows x 33 channels.
template <int DT>
void launch_channel_embedding(dim3 grid, int threads, hipStream_t s, const ChannelEmbeddingParams& p) {
  if (threads == 64)
    hipLaunchKernelGGL((channel_embedding_sum_kernel<DT, 16>), grid, dim3(threads), 0, s, p);
  else
    hipLaunchKernelGGL((channel_embedding_sum_kernel<DT, 2>), grid, dim3(threads), 0, s, p);
}

}  // namespace

extern "C" int omni_channel_embedding_sum(const void* token_ids, int ids_dtype, int64_t rows,
                                          int64_t channels, int64_t id_stride_row,
                                          int64_t id_stride_channel, const uint64_t* tables,
                                          const int64_t* vocab_sizes, int dtype, int64_t hidden,
                                          void* out, omni_stream_t stream) {
  if (!token_ids || !tables || !vocab_sizes || !out) return OMNI_ERR_INVALID_ARG;
  if (ids_dtype != OMNI_DTYPE_I32 && ids_dtype != OMNI_DTYPE_I64) return OMNI_ERR_INVALID_ARG;
  if (dtype != OMNI_DTYPE_BF16 && dtype != OMNI_DTYPE_F16 && dtype != OMNI_DTYPE_F32)
    return OMNI_ERR_INVALID_ARG;
  if (rows < 0 || channels < 1 || hidden < 1) return OMNI_ERR_INVALID_ARG;
  if (rows == 0) return OMNI_OK;
  // 256-thread workgroups, or 64-thread ones when that leaves fewer than two per CU (decode
  // batches of a few dozen rows)
  int threads = kThreads;
  if (rows * ((hidden + kThreads * kCols - 1) / (kThreads * kCols)) < 512) threads = 64;
  const int64_t per_block = (int64_t)threads * kCols;
  const int64_t col_blocks = (hidden + per_block - 1) / per_block;
  if (channels > 0x7fffffff || rows * col_blocks > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  ChannelEmbeddingParams p{token_ids, ids_dtype, id_stride_row, id_stride_channel, (int)channels,
                           tables, vocab_sizes, hidden, out, col_blocks,
                           (reinterpret_cast<uintptr_t>(out) & 15) == 0};
  dim3 grid((unsigned)(rows * col_blocks));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == OMNI_DTYPE_BF16)
    launch_channel_embedding<OMNI_DTYPE_BF16>(grid, threads, s, p);
  else if (dtype == OMNI_DTYPE_F16)
    launch_channel_embedding<OMNI_DTYPE_F16>(grid, threads, s, p);
  else
    launch_channel_embedding<OMNI_DTYPE_F32>(grid, threads, s, p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}
