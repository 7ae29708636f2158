// The Qwen3-Omni code2wav front on gfx950: every op of the pre-transformer and the ConvNeXt
// upsamplers that is not a plain GEMM (the GEMMs are hipBLASLt calls between these launches).
//
//   rms_norm_residual_kernel   h += scale * delta (layer scale + residual, float32 h), then
//                              normed = RMSNorm(h) * weight as the next GEMM's bf16 operand
//                              (code2wav.py:300-324's addcmul + rmsnorm; the layer's input norm)
//   rope_kv_kernel             neox rotary on q and k in the qkv GEMM output, in place, at the
//                              rows' absolute positions, and the new K / V into the slots' rings
//                              (apply_rope_inplace_with_kvcache, code2wav.py:205-215)
//   window_attention_kernel    causal sliding-window softmax attention of the new frames over
//                              their window (rows' rings or, for a stream's first decode, the
//                              qkv buffer itself) on MFMA (code2wav.py:227-246,278-298)
//   silu_mul_kernel            silu(gate) * up of the merged gate / up GEMM (code2wav.py:318)
//   dwconv_layernorm_kernel    ConvNeXt's depthwise causal conv (k = 7) over the float32
//                              residual stream with per-slot history, then LayerNorm, as the
//                              first MLP GEMM's bf16 operand (incremental_codec.py:160-175)
//   bias_gelu_kernel           GELU(y + b) in place (erf form, nn.GELU())
//   bias_scale_residual_kernel r += gamma * (y + b), and the next conv's bf16 operand
//   advance_positions_kernel   frame_positions[slot] = start + new frames (code2wav.py:459)
//
// One wave per row wherever a row is reduced (RMSNorm, LayerNorm): the channels sit in
// registers, 4 per lane per 256-channel group, and the reduction is a wave shuffle.
#include "common.h"
#include "rope.h"

namespace {

constexpr int kWave = 64;

OMNI_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

OMNI_DEVICE float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

OMNI_DEVICE void load_bf16x4(const u16* p, float v[4]) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  v[0] = __uint_as_float(w.x << 16);
  v[1] = __uint_as_float(w.x & 0xffff0000u);
  v[2] = __uint_as_float(w.y << 16);
  v[3] = __uint_as_float(w.y & 0xffff0000u);
}

OMNI_DEVICE void store_bf16x4(u16* p, const float v[4]) {
  uint2 w;
  w.x = (uint32_t)float_to_bits_bf16(v[0]) | ((uint32_t)float_to_bits_bf16(v[1]) << 16);
  w.y = (uint32_t)float_to_bits_bf16(v[2]) | ((uint32_t)float_to_bits_bf16(v[3]) << 16);
  *reinterpret_cast<uint2*>(p) = w;
}

OMNI_DEVICE void load_bf16x8(const u16* p, float v[8]) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(a[i] << 16);
    v[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
  }
}

OMNI_DEVICE void store_bf16x8(u16* p, const float v[8]) {
  uint4 w;
  w.x = (uint32_t)float_to_bits_bf16(v[0]) | ((uint32_t)float_to_bits_bf16(v[1]) << 16);
  w.y = (uint32_t)float_to_bits_bf16(v[2]) | ((uint32_t)float_to_bits_bf16(v[3]) << 16);
  w.z = (uint32_t)float_to_bits_bf16(v[4]) | ((uint32_t)float_to_bits_bf16(v[5]) << 16);
  w.w = (uint32_t)float_to_bits_bf16(v[6]) | ((uint32_t)float_to_bits_bf16(v[7]) << 16);
  *reinterpret_cast<uint4*>(p) = w;
}

// ------------------------------------------------------------------------------ RMSNorm

constexpr int kMaxGroups = 16;  // channels <= 16 * 256

struct RmsParams {
  float* h;
  int64_t rows;
  int channels;
  int groups;  // channels / 256
  const u16* delta;
  int64_t delta_stride;
  const float* scale;
  const float* weight;
  float eps;
  u16* normed;
  int64_t normed_stride;
};

// One wave per row. Every load of the row (h, and the weights) is issued before the first use
// of any of them, and the residual add's stores come after all of them: a store into h between
// two groups' loads would keep the compiler from moving the later loads above it, one memory
// round trip per 256-channel group. GROUPS > 0 fixes the group count (unrolled, no guards);
// GROUPS = 0 reads it from p.groups. The sum of squares runs group by group, element by element,
// in both forms.
template <int GROUPS>
__global__ __launch_bounds__(256) void rms_norm_residual_kernel(RmsParams p) {
  constexpr int NG = GROUPS > 0 ? GROUPS : kMaxGroups;
  const int groups = GROUPS > 0 ? GROUPS : p.groups;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  float* hr = p.h + row * p.channels;
  f32x4 x[NG], w[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (GROUPS > 0 || g < groups) {
      const int c = (g * kWave + lane) * 4;
      x[g] = *reinterpret_cast<const f32x4*>(hr + c);
      w[g] = *reinterpret_cast<const f32x4*>(p.weight + c);
    }
  }
  if (p.delta) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (GROUPS > 0 || g < groups) {
        const int c = (g * kWave + lane) * 4;
        float d[4];
        load_bf16x4(p.delta + row * p.delta_stride + c, d);
        const f32x4 sc = *reinterpret_cast<const f32x4*>(p.scale + c);
#pragma unroll
        for (int k = 0; k < 4; ++k) x[g][k] += sc[k] * d[k];
      }
    }
#pragma unroll
    for (int g = 0; g < NG; ++g)
      if (GROUPS > 0 || g < groups)
        *reinterpret_cast<f32x4*>(hr + (g * kWave + lane) * 4) = x[g];
  }
  float ss = 0.f;
#pragma unroll
  for (int g = 0; g < NG; ++g)
    if (GROUPS > 0 || g < groups)
#pragma unroll
      for (int k = 0; k < 4; ++k) ss += x[g][k] * x[g][k];
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)p.channels + p.eps);
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (GROUPS > 0 || g < groups) {
      const int c = (g * kWave + lane) * 4;
      const float o[4] = {w[g][0] * (x[g][0] * inv), w[g][1] * (x[g][1] * inv),
                          w[g][2] * (x[g][2] * inv), w[g][3] * (x[g][3] * inv)};
      store_bf16x4(p.normed + row * p.normed_stride + c, o);
    }
  }
}

// ------------------------------------------------------------------------------ rotary + rings

struct RopeParams {
  u16* qkv;
  int64_t frames;  // T, rows per batch row
  int64_t qkv_stride;
  int heads, kv_heads, head_dim;
  const float* inv_freq;  // [head_dim / 2]
  const int64_t* slot_index;
  const int64_t* positions;
  int cold;
  int64_t num_slots;
  u16* key_ring;
  u16* value_ring;
  int64_t ring_frames;
};

// One workgroup per token (b * T + t): the rotary pairs of its q and k heads, then its V row
// into the ring.
__global__ __launch_bounds__(256) void rope_kv_kernel(RopeParams p) {
  const int64_t token = blockIdx.x;
  const int64_t b = token / p.frames;
  const int64_t t = token - b * p.frames;
  int64_t slot;
  const int64_t pos = row_start(p.slot_index, p.positions, p.cold, p.num_slots, b, &slot) + t;
  u16* row = p.qkv + token * p.qkv_stride;
  const int half = p.head_dim / 2;
  const int kv_width = p.kv_heads * p.head_dim;
  const bool ring = p.key_ring != nullptr && slot >= 0;
  const int64_t ring_row = ring ? slot * p.ring_frames + pos % p.ring_frames : 0;
  const int pairs = (p.heads + p.kv_heads) * half;
  const float fpos = (float)pos;
  for (int item = threadIdx.x; item < pairs; item += blockDim.x) {
    const int head = item / half;
    const int i = item - head * half;
    const int col = head * p.head_dim + i;  // q heads, then k heads, are contiguous
    u16 y1, y2;
    rope_pair(bits_to_float_bf16(row[col]), bits_to_float_bf16(row[col + half]),
              fpos * p.inv_freq[i], &y1, &y2);
    row[col] = y1;
    row[col + half] = y2;
    if (ring && head >= p.heads) {
      u16* k = p.key_ring + ring_row * kv_width + (col - p.heads * p.head_dim);
      k[0] = y1;
      k[half] = y2;
    }
  }
  if (ring) {
    const u16* v = row + (p.heads + p.kv_heads) * p.head_dim;
    u16* dst = p.value_ring + ring_row * kv_width;
    for (int e = threadIdx.x; e < kv_width; e += blockDim.x) dst[e] = v[e];
  }
}

// ------------------------------------------------------------------------------ attention
//
// One wave per (batch row, head, tile of 16 queries), both products on v_mfma_f32_16x16x32_bf16:
//   S^T = K Q^T   (M = 16 keys per tile, N = 16 queries, K = 64 dims in two steps)
//   O^T = V^T P^T (M = 16 dims per tile, N = 16 queries, K = 32 keys per step)
// Lane l = 16 g + n holds S^T[key 4 g + e][query n] of each key tile (e < 4). The softmax of
// query n reduces over the lane's registers and the 4 lanes n, n + 16, n + 32, n + 48. For the
// second product the lane's probabilities go in as they lie: K-step s takes, in lane (g, n), the
// keys 32 s + 4 g + (0..3) of tile 2 s and 32 s + 16 + 4 g + (0..3) of tile 2 s + 1, and V^T is
// read from LDS in that same key order, so the keys' order in the sum is a fixed permutation and
// no probability crosses lanes. P is rounded to bf16 for the product; everything else is float32.

constexpr int kQueries = 16;     // queries per wave
constexpr int kHeadDim = 64;
constexpr int kMaxKeyTiles = 8;  // 16-key tiles: window - 1 + 16 <= 128 keys
constexpr int kKRow = kHeadDim + 16;  // bf16 pitch of a K row in LDS: 10 16-byte slots, a pitch
                                      // of 2 mod 4 slots, at which 16-row reads meet no bank conflict

struct AttnParams {
  const u16* qkv;
  int64_t frames;
  int64_t qkv_stride;
  int heads, kv_heads;
  int window;
  float scale_log2;  // softmax scale times log2(e): p = 2^(s * scale_log2 - max)
  const u16* key_ring;  // null: keys and values come from qkv (a first decode)
  const u16* value_ring;
  int64_t ring_frames;
  const int64_t* slot_index;
  const int64_t* positions;
  int cold;
  int64_t num_slots;
  u16* out;
  int64_t out_stride;
  int key_slots;  // keys staged per wave: a multiple of 32 >= window - 1 + 16
};

size_t attention_lds_bytes(int key_slots) {
  // K [key_slots][kKRow] and V^T [64][key_slots + 8], bf16
  return 2 * ((size_t)key_slots * kKRow + (size_t)kHeadDim * (key_slots + 8));
}

__global__ __launch_bounds__(64) void window_attention_kernel(AttnParams p) {
  extern __shared__ u16 alds[];
  const int64_t b = blockIdx.z;
  const int head = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * kQueries;
  const int kvh = head / (p.heads / p.kv_heads);
  const int lane = threadIdx.x;
  const int ks_n = p.key_slots;
  const int vpitch = ks_n + 8;
  u16* ks = alds;                              // [ks_n][kKRow]
  u16* vt = alds + (size_t)ks_n * kKRow;       // [64][vpitch]
  int64_t slot;
  const int64_t start = row_start(p.slot_index, p.positions, p.cold, p.num_slots, b, &slot);
  const bool ring = p.key_ring != nullptr;
  const int64_t p0 = start + t0;
  const int64_t last_t = min(t0 + kQueries, p.frames) - 1;
  const int64_t kp0 = max(p0 - (p.window - 1), (int64_t)0);
  const int nk = (int)(start + last_t - kp0 + 1);  // <= window - 1 + 16 <= ks_n
  const int kv_width = p.kv_heads * kHeadDim;
  // stage K (row-major) and V (transposed), 8 bf16 per lane and step; rows >= nk are zeros.
  // Every step's loads are issued before the first LDS store, so the staging waits on one
  // round trip to memory instead of one per step.
  constexpr int kMaxSteps = kMaxKeyTiles * 16 * (kHeadDim / 8) / kWave;
  uint4 kw[kMaxSteps], vw[kMaxSteps];
  {
    // ring row of key row r = lane / 8 + 8 i: (kp0 + r) mod ring_frames, advanced by 8 a step
    // (ring_frames >= window - 1 + frames > 8)
    const int rf = (int)p.ring_frames;
    int rr = ring ? (int)((kp0 + (lane >> 3)) % p.ring_frames) : 0;
#pragma unroll
    for (int i = 0; i < kMaxSteps; ++i) {
      const int e = lane + i * kWave;
      const int r = e >> 3;
      const int c8 = (e & 7) * 8;
      kw[i] = make_uint4(0, 0, 0, 0);
      vw[i] = kw[i];
      if (e < ks_n * (kHeadDim / 8) && r < nk) {
        const u16* ksrc;
        const u16* vsrc;
        if (ring) {
          const int64_t row = (slot < 0 ? 0 : slot) * p.ring_frames + rr;
          ksrc = p.key_ring + row * kv_width + kvh * kHeadDim + c8;
          vsrc = p.value_ring + row * kv_width + kvh * kHeadDim + c8;
        } else {
          const u16* tok = p.qkv + (b * p.frames + (kp0 + r - start)) * p.qkv_stride;
          ksrc = tok + (p.heads + kvh) * kHeadDim + c8;
          vsrc = tok + (p.heads + p.kv_heads + kvh) * kHeadDim + c8;
        }
        kw[i] = *reinterpret_cast<const uint4*>(ksrc);
        vw[i] = *reinterpret_cast<const uint4*>(vsrc);
      }
      if (ring) {
        rr += 8;
        if (rr >= rf) rr -= rf;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kMaxSteps; ++i) {
    const int e = lane + i * kWave;
    if (e < ks_n * (kHeadDim / 8)) {
      const int r = e >> 3;
      const int c8 = (e & 7) * 8;
      *reinterpret_cast<uint4*>(ks + r * kKRow + c8) = kw[i];
      const uint32_t vv[4] = {vw[i].x, vw[i].y, vw[i].z, vw[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vt[(c8 + 2 * j) * vpitch + r] = (u16)(vv[j] & 0xffff);
        vt[(c8 + 2 * j + 1) * vpitch + r] = (u16)(vv[j] >> 16);
      }
    }
  }
  // this lane's query row n (zeros past the last query) as the B operand, dims 8 g .. 8 g + 7
  // and 32 + 8 g ..
  const int n = lane & 15;
  const int g = lane >> 4;
  const int nq = (int)(last_t - t0 + 1);
  bf16x8 qv[2];
  {
    uint4 w0 = make_uint4(0, 0, 0, 0), w1 = w0;
    if (n < nq) {
      const u16* q = p.qkv + (b * p.frames + t0 + n) * p.qkv_stride + head * kHeadDim + 8 * g;
      w0 = *reinterpret_cast<const uint4*>(q);
      w1 = *reinterpret_cast<const uint4*>(q + 32);
    }
    qv[0] = *reinterpret_cast<const bf16x8*>(&w0);
    qv[1] = *reinterpret_cast<const bf16x8*>(&w1);
  }
  __syncthreads();
  const int tiles = (nk + 15) / 16;
  f32x4 st[kMaxKeyTiles];
  const int64_t qpos = p0 + n;
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < kMaxKeyTiles; ++t) {
    if (t < tiles) {
      const u16* krow = ks + (16 * t + n) * kKRow + 8 * g;  // A: key row (lane & 15)
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8*>(krow),
                                                    qv[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8*>(krow + 32),
                                                    qv[1], acc, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = 16 * t + 4 * g + e;
        const int64_t d = qpos - (kp0 + key);
        const bool ok = key < nk && d >= 0 && d < p.window;
        acc[e] = ok ? acc[e] * p.scale_log2 : -INFINITY;
        m = fmaxf(m, acc[e]);
      }
      st[t] = acc;
    } else {
      st[t] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
  }
  m = fmaxf(m, __shfl_xor(m, 16, kWave));
  m = fmaxf(m, __shfl_xor(m, 32, kWave));
  if (m == -INFINITY) m = 0.f;  // a padding query (no stored output)
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < kMaxKeyTiles; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pe = t < tiles ? __builtin_amdgcn_exp2f(st[t][e] - m) : 0.f;
      st[t][e] = pe;
      sum += pe;
    }
  sum += __shfl_xor(sum, 16, kWave);
  sum += __shfl_xor(sum, 32, kWave);
  // O^T = V^T P^T over K-steps of 32 keys
  f32x4 o[kHeadDim / 16];
#pragma unroll
  for (int dt = 0; dt < kHeadDim / 16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < kMaxKeyTiles / 2; ++s2) {
    if (2 * s2 < tiles) {
      bf16x8 pb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pb[e] = to_bf16(st[2 * s2][e]);
        pb[4 + e] = to_bf16(st[2 * s2 + 1][e]);
      }
      const int k0 = 32 * s2 + 4 * g;
#pragma unroll
      for (int dt = 0; dt < kHeadDim / 16; ++dt) {
        const u16* vrow = vt + (16 * dt + n) * vpitch;  // A: dim row (lane & 15)
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + k0);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + k0 + 16);
        const uint4 w = make_uint4(lo.x, lo.y, hi.x, hi.y);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8*>(&w), pb,
                                                        o[dt], 0, 0, 0);
      }
    }
  }
  if (n < nq) {
    const float inv = 1.f / sum;
    u16* dst = p.out + (b * p.frames + t0 + n) * p.out_stride + head * kHeadDim + 4 * g;
#pragma unroll
    for (int dt = 0; dt < kHeadDim / 16; ++dt) {
      const float v[4] = {o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv};
      store_bf16x4(dst + 16 * dt, v);
    }
  }
}

// ------------------------------------------------------------------------------ SwiGLU

struct SiluMulParams {
  const u16* gate_up;
  int64_t rows;
  int64_t inter;
  int64_t in_stride;
  u16* out;
  int64_t out_stride;
};

__global__ __launch_bounds__(256) void silu_mul_kernel(SiluMulParams p) {
  const int64_t per_row = p.inter / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.rows * per_row) return;
  const int64_t row = idx / per_row;
  const int64_t c = (idx - row * per_row) * 8;
  float g[8], u[8], o[8];
  load_bf16x8(p.gate_up + row * p.in_stride + c, g);
  load_bf16x8(p.gate_up + row * p.in_stride + p.inter + c, u);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = g[i] / (1.f + __expf(-g[i])) * u[i];
  store_bf16x8(p.out + row * p.out_stride + c, o);
}

// ------------------------------------------------------------------------------ ConvNeXt

constexpr int kDwTaps = 7;
constexpr int kDwHistory = kDwTaps - 1;

struct DwParams {
  const float* x;  // [B][L][C] float32, rows x_stride_b apart
  int64_t x_stride_b;
  int64_t length;
  int channels;
  int groups;
  const float* weight;  // [7][C]
  const float* bias;
  const float* ln_weight;
  const float* ln_bias;
  float eps;
  float* hist;  // [slots][2][6][C] float32 (nullable)
  int64_t hist_slot_stride;
  const int64_t* slot_index;
  const int64_t* slot_parity;
  int64_t num_slots;
  int cold;
  u16* out;  // [B][L][C] bf16, rows out_stride_b apart
  int64_t out_stride_b;
  int pos_blocks;  // workgroups of positions per batch row (one more writes the new history)
};

// GROUPS > 0 fixes the 256-channel group count (unrolled, the groups' loads issued together);
// GROUPS = 0 reads it from p.groups.
template <int GROUPS>
__global__ __launch_bounds__(256) void dwconv_layernorm_kernel(DwParams p) {
  constexpr int NG = GROUPS > 0 ? GROUPS : kMaxGroups;
  const int groups = GROUPS > 0 ? GROUPS : p.groups;
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int C = p.channels;
  int64_t slot = -1;
  if (p.hist && p.slot_index) {
    slot = p.slot_index[b];
    if (slot < 0 || slot >= p.num_slots) slot = -1;
  }
  const int parity = slot >= 0 ? (int)(p.slot_parity[slot] & 1) : 0;
  const float* hread =
      (slot >= 0 && !p.cold) ? p.hist + slot * p.hist_slot_stride + parity * kDwHistory * C
                             : nullptr;
  const float* xb = p.x + b * p.x_stride_b;
  // this row's samples and its slot's old history as buffers (the launcher keeps a row's
  // samples under 2 GiB); without a history its buffer is empty and reads zeros
  const auto x_rsrc = buffer_rsrc(xb, (uint32_t)(p.length * C * 4));
  const auto h_rsrc = buffer_rsrc(hread, hread ? (uint32_t)(kDwHistory * C * 4) : 0u);
  if ((int)blockIdx.x == p.pos_blocks) {
    // the new history: the last 6 samples of (old history ++ this call's samples); every load
    // before the first store (one at a time, each waited on, they were the launch's longest path)
    if (slot < 0) return;
    float* hw = p.hist + slot * p.hist_slot_stride + (1 - parity) * kDwHistory * C;
    auto source = [&](int e) {
      const int s = e / C;
      const int c = e - s * C;
      const int q = (int)p.length + s;  // index into (history ++ samples)
      const uint32_t xo = q >= kDwHistory ? (uint32_t)((q - kDwHistory) * C + c) * 4u : kOutOfRange;
      const uint32_t ho = q < kDwHistory ? (uint32_t)(q * C + c) * 4u : kOutOfRange;
      return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x_rsrc, xo, 0, 0) |
                                           __builtin_amdgcn_raw_buffer_load_b32(h_rsrc, ho, 0, 0));
    };
    if constexpr (GROUPS > 0) {
      constexpr int PER = kDwHistory * GROUPS;  // kDwHistory * C / 256 elements a thread
      float hv[PER];
#pragma unroll
      for (int u = 0; u < PER; ++u) hv[u] = source((int)threadIdx.x + u * 256);
#pragma unroll
      for (int u = 0; u < PER; ++u) hw[threadIdx.x + u * 256] = hv[u];
    } else {
      for (int e = threadIdx.x; e < kDwHistory * C; e += blockDim.x) hw[e] = source(e);
    }
    return;
  }
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= p.length) return;
  float v[NG][4];
  float sum = 0.f;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (GROUPS > 0 || g < groups) {
      const int c = (g * kWave + lane) * 4;
      const float4 bias = *reinterpret_cast<const float4*>(p.bias + c);
      float a[4] = {bias.x, bias.y, bias.z, bias.w};
      // the group's 7 taps and 7 weight vectors loaded into arrays before the first product:
      // both sources of a tap loaded unconditionally, the one that does not hold it (or both,
      // for a zero) at an out-of-range offset that reads zeros (loads under branches, or into
      // one reused register, were issued one tap at a time)
      float4 xt[kDwTaps], wt[kDwTaps];
#pragma unroll
      for (int j = 0; j < kDwTaps; ++j) {
        const int pos = (int)t - kDwHistory + j;
        const uint32_t xo = pos >= 0 ? (uint32_t)(pos * C + c) * 4u : kOutOfRange;
        const uint32_t ho = pos < 0 ? (uint32_t)((kDwHistory + pos) * C + c) * 4u : kOutOfRange;
        xt[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, xo, 0, 0) |
                                               __builtin_amdgcn_raw_buffer_load_b128(h_rsrc, ho, 0, 0));
        wt[j] = *reinterpret_cast<const float4*>(p.weight + j * C + c);
      }
#pragma unroll
      for (int j = 0; j < kDwTaps; ++j) {
        a[0] += wt[j].x * xt[j].x;
        a[1] += wt[j].y * xt[j].y;
        a[2] += wt[j].z * xt[j].z;
        a[3] += wt[j].w * xt[j].w;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[g][k] = a[k];
        sum += a[k];
      }
    }
  }
  const float mean = wave_sum(sum) / (float)C;
  float var = 0.f;
#pragma unroll
  for (int g = 0; g < NG; ++g)
    if (GROUPS > 0 || g < groups)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float d = v[g][k] - mean;
        var += d * d;
      }
  const float inv = rsqrtf(wave_sum(var) / (float)C + p.eps);
  u16* ob = p.out + b * p.out_stride_b + t * C;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (GROUPS > 0 || g < groups) {
      const int c = (g * kWave + lane) * 4;
      const float4 w = *reinterpret_cast<const float4*>(p.ln_weight + c);
      const float4 bb = *reinterpret_cast<const float4*>(p.ln_bias + c);
      const float o[4] = {(v[g][0] - mean) * inv * w.x + bb.x, (v[g][1] - mean) * inv * w.y + bb.y,
                          (v[g][2] - mean) * inv * w.z + bb.z, (v[g][3] - mean) * inv * w.w + bb.w};
      store_bf16x4(ob + c, o);
    }
  }
}

struct BiasGeluParams {
  u16* y;
  int64_t rows, cols, stride;
  const float* bias;
};

__global__ __launch_bounds__(256) void bias_gelu_kernel(BiasGeluParams p) {
  const int64_t per_row = p.cols / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.rows * per_row) return;
  const int64_t row = idx / per_row;
  const int64_t c = (idx - row * per_row) * 8;
  u16* ptr = p.y + row * p.stride + c;
  float v[8];
  load_bf16x8(ptr, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float x = v[i] + p.bias[c + i];
    v[i] = 0.5f * x * (1.f + erff(x * 0.70710678118654752f));
  }
  store_bf16x8(ptr, v);
}

struct ScaleResidualParams {
  float* r;  // [rows][channels] float32, contiguous
  int64_t rows;
  int64_t channels;
  const u16* y;
  int64_t y_stride;
  const float* bias;
  const float* gamma;
  u16* out;  // bf16 copy of the new r (nullable)
  int64_t out_stride;
};

__global__ __launch_bounds__(256) void bias_scale_residual_kernel(ScaleResidualParams p) {
  const int64_t per_row = p.channels / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.rows * per_row) return;
  const int64_t row = idx / per_row;
  const int64_t c = (idx - row * per_row) * 4;
  float* rp = p.r + row * p.channels + c;
  float4 r = *reinterpret_cast<float4*>(rp);
  float y[4];
  load_bf16x4(p.y + row * p.y_stride + c, y);
  const float4 b = *reinterpret_cast<const float4*>(p.bias + c);
  const float4 g = *reinterpret_cast<const float4*>(p.gamma + c);
  r.x += g.x * (y[0] + b.x);
  r.y += g.y * (y[1] + b.y);
  r.z += g.z * (y[2] + b.z);
  r.w += g.w * (y[3] + b.w);
  *reinterpret_cast<float4*>(rp) = r;
  if (p.out) {
    const float o[4] = {r.x, r.y, r.z, r.w};
    store_bf16x4(p.out + row * p.out_stride + c, o);
  }
}

__global__ void advance_positions_kernel(int64_t* positions, int64_t num_slots,
                                         const int64_t* slot_index, int64_t rows,
                                         int64_t new_frames, int cold) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int64_t slot = slot_index[r];
  if (slot < 0 || slot >= num_slots) return;
  positions[slot] = (cold ? 0 : positions[slot]) + new_frames;
}

bool aligned(const void* ptr, int bytes) {
  return (reinterpret_cast<uintptr_t>(ptr) & (uintptr_t)(bytes - 1)) == 0;
}

unsigned blocks_for(int64_t items, int threads) { return (unsigned)((items + threads - 1) / threads); }

}  // namespace

extern "C" int omni_rms_norm_residual(float* h, int64_t rows, int64_t channels, const void* delta,
                                      int64_t delta_stride, const float* scale,
                                      const float* weight, float eps, void* normed,
                                      int64_t normed_stride, omni_stream_t stream) {
  if (!h || !weight || !normed || rows < 0) return OMNI_ERR_INVALID_ARG;
  if (channels < 256 || channels % 256 || channels > 256 * kMaxGroups) return OMNI_ERR_UNSUPPORTED;
  if (delta && (!scale || delta_stride < channels || delta_stride % 4)) return OMNI_ERR_INVALID_ARG;
  if (normed_stride < channels || normed_stride % 4 || !(eps >= 0.f)) return OMNI_ERR_INVALID_ARG;
  if (!aligned(h, 16) || !aligned(normed, 8) || (delta && !aligned(delta, 8)))
    return OMNI_ERR_INVALID_ARG;
  if (rows == 0) return OMNI_OK;
  RmsParams p{h, rows, (int)channels, (int)(channels / 256), static_cast<const u16*>(delta),
              delta_stride, scale, weight, eps, static_cast<u16*>(normed), normed_stride};
  // 1024 channels (the code2wav pre-transformers' hidden size) unrolled, others generic
  hipLaunchKernelGGL(p.groups == 4 ? rms_norm_residual_kernel<4> : rms_norm_residual_kernel<0>,
                     dim3(blocks_for(rows, 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_rope_kv_write(void* qkv, int64_t batch, int64_t frames, int64_t qkv_stride,
                                  int64_t heads, int64_t kv_heads, int64_t head_dim,
                                  const float* inv_freq, const int64_t* slot_index,
                                  const int64_t* positions, int cold, int64_t num_slots,
                                  void* key_ring, void* value_ring, int64_t ring_frames,
                                  omni_stream_t stream) {
  if (!qkv || !inv_freq || batch < 0 || frames < 0) return OMNI_ERR_INVALID_ARG;
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 2 || head_dim % 2)
    return OMNI_ERR_INVALID_ARG;
  if (qkv_stride < (heads + 2 * kv_heads) * head_dim) return OMNI_ERR_INVALID_ARG;
  if ((key_ring != nullptr) != (value_ring != nullptr)) return OMNI_ERR_INVALID_ARG;
  if (key_ring && (!slot_index || ring_frames < 1)) return OMNI_ERR_INVALID_ARG;
  if (!cold && (!slot_index || !positions)) return OMNI_ERR_INVALID_ARG;
  if (batch * frames == 0) return OMNI_OK;
  if (batch * frames > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  RopeParams p{static_cast<u16*>(qkv), frames, qkv_stride, (int)heads, (int)kv_heads,
               (int)head_dim, inv_freq, slot_index, positions, cold, num_slots,
               static_cast<u16*>(key_ring), static_cast<u16*>(value_ring), ring_frames};
  hipLaunchKernelGGL(rope_kv_kernel, dim3((unsigned)(batch * frames)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_window_attention(const void* qkv, int64_t batch, int64_t frames,
                                     int64_t qkv_stride, int64_t heads, int64_t kv_heads,
                                     int64_t head_dim, int64_t window, float scale,
                                     const void* key_ring, const void* value_ring,
                                     int64_t ring_frames, const int64_t* slot_index,
                                     const int64_t* positions, int cold, int64_t num_slots,
                                     void* out, int64_t out_stride, omni_stream_t stream) {
  if (!qkv || !out || batch < 0 || frames < 0) return OMNI_ERR_INVALID_ARG;
  if (heads < 1 || kv_heads < 1 || heads % kv_heads) return OMNI_ERR_INVALID_ARG;
  if (head_dim != kHeadDim) return OMNI_ERR_UNSUPPORTED;
  if (window < 1) return OMNI_ERR_INVALID_ARG;
  if (qkv_stride < (heads + 2 * kv_heads) * head_dim || qkv_stride % 8 ||
      out_stride < heads * head_dim || out_stride % 4)
    return OMNI_ERR_INVALID_ARG;
  if (!aligned(qkv, 16) || !aligned(out, 8)) return OMNI_ERR_INVALID_ARG;
  if ((key_ring != nullptr) != (value_ring != nullptr)) return OMNI_ERR_INVALID_ARG;
  if (key_ring) {
    // the ring holds the window before the new frames and the frames themselves
    if (!slot_index || ring_frames < window - 1 + frames) return OMNI_ERR_INVALID_ARG;
    if (!aligned(key_ring, 16) || !aligned(value_ring, 16)) return OMNI_ERR_INVALID_ARG;
    if (!cold && !positions) return OMNI_ERR_INVALID_ARG;
  } else if (!cold) {
    return OMNI_ERR_INVALID_ARG;  // without rings only a stream's first frames have their keys
  }
  if (batch * frames == 0) return OMNI_OK;
  if (batch > 65535 || heads > 65535) return OMNI_ERR_UNSUPPORTED;
  const int key_slots = (int)((window - 1 + kQueries + 31) / 32 * 32);
  if (key_slots > 16 * kMaxKeyTiles) return OMNI_ERR_UNSUPPORTED;
  AttnParams p{static_cast<const u16*>(qkv), frames, qkv_stride, (int)heads, (int)kv_heads,
               (int)window, scale * 1.4426950408889634f, static_cast<const u16*>(key_ring),
               static_cast<const u16*>(value_ring), ring_frames, slot_index, positions, cold,
               num_slots, static_cast<u16*>(out), out_stride, key_slots};
  const size_t lds = attention_lds_bytes(key_slots);
  dim3 grid(blocks_for(frames, kQueries), (unsigned)heads, (unsigned)batch);
  hipLaunchKernelGGL(window_attention_kernel, grid, dim3(kWave), lds,
                     reinterpret_cast<hipStream_t>(stream), p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_silu_mul(const void* gate_up, int64_t rows, int64_t inter, int64_t in_stride,
                             void* out, int64_t out_stride, omni_stream_t stream) {
  if (!gate_up || !out || rows < 0 || inter < 8 || inter % 8) return OMNI_ERR_INVALID_ARG;
  if (in_stride < 2 * inter || in_stride % 8 || out_stride < inter || out_stride % 8)
    return OMNI_ERR_INVALID_ARG;
  if (!aligned(gate_up, 16) || !aligned(out, 16)) return OMNI_ERR_INVALID_ARG;
  if (rows == 0) return OMNI_OK;
  SiluMulParams p{static_cast<const u16*>(gate_up), rows, inter, in_stride,
                  static_cast<u16*>(out), out_stride};
  hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_for(rows * (inter / 8), 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_dwconv_layernorm(const float* x, int64_t batch, int64_t length,
                                     int64_t channels, int64_t x_stride_b, const float* weight,
                                     const float* bias, const float* ln_weight,
                                     const float* ln_bias, float eps, float* hist_pool,
                                     int64_t hist_slot_stride, const int64_t* slot_index,
                                     const int64_t* slot_parity, int64_t num_slots, int cold,
                                     void* out, int64_t out_stride_b, omni_stream_t stream) {
  if (!x || !weight || !bias || !ln_weight || !ln_bias || !out) return OMNI_ERR_INVALID_ARG;
  if (batch < 0 || length < 0) return OMNI_ERR_INVALID_ARG;
  if (channels < 256 || channels % 256 || channels > 256 * kMaxGroups) return OMNI_ERR_UNSUPPORTED;
  if (x_stride_b < length * channels || x_stride_b % 4 || out_stride_b < length * channels ||
      out_stride_b % 4)
    return OMNI_ERR_INVALID_ARG;
  if (hist_pool && (!slot_index || !slot_parity || hist_slot_stride < 2 * kDwHistory * channels))
    return OMNI_ERR_INVALID_ARG;
  if (!aligned(x, 16) || !aligned(out, 8) || (hist_pool && !aligned(hist_pool, 16)))
    return OMNI_ERR_INVALID_ARG;
  if (batch == 0 || length == 0) return OMNI_OK;
  if (batch > 65535 || length * channels * 4 > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  DwParams p{};
  p.x = x;
  p.x_stride_b = x_stride_b;
  p.length = length;
  p.channels = (int)channels;
  p.groups = (int)(channels / 256);
  p.weight = weight;
  p.bias = bias;
  p.ln_weight = ln_weight;
  p.ln_bias = ln_bias;
  p.eps = eps;
  p.hist = hist_pool;
  p.hist_slot_stride = hist_slot_stride;
  p.slot_index = slot_index;
  p.slot_parity = slot_parity;
  p.num_slots = num_slots;
  p.cold = cold;
  p.out = static_cast<u16*>(out);
  p.out_stride_b = out_stride_b;
  p.pos_blocks = (int)blocks_for(length, 4);
  dim3 grid((unsigned)(p.pos_blocks + 1), (unsigned)batch);
  hipLaunchKernelGGL(p.groups == 4 ? dwconv_layernorm_kernel<4> : dwconv_layernorm_kernel<0>,
                     grid, dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_bias_gelu(void* y, int64_t rows, int64_t cols, int64_t stride,
                              const float* bias, omni_stream_t stream) {
  if (!y || !bias || rows < 0 || cols < 8 || cols % 8 || stride < cols || stride % 8)
    return OMNI_ERR_INVALID_ARG;
  if (!aligned(y, 16)) return OMNI_ERR_INVALID_ARG;
  if (rows == 0) return OMNI_OK;
  BiasGeluParams p{static_cast<u16*>(y), rows, cols, stride, bias};
  hipLaunchKernelGGL(bias_gelu_kernel, dim3(blocks_for(rows * (cols / 8), 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_bias_scale_residual(float* r, int64_t rows, int64_t channels, const void* y,
                                        int64_t y_stride, const float* bias, const float* gamma,
                                        void* out, int64_t out_stride, omni_stream_t stream) {
  if (!r || !y || !bias || !gamma || rows < 0 || channels < 4 || channels % 4)
    return OMNI_ERR_INVALID_ARG;
  if (y_stride < channels || y_stride % 4 || (out && (out_stride < channels || out_stride % 4)))
    return OMNI_ERR_INVALID_ARG;
  if (!aligned(r, 16) || !aligned(y, 8) || !aligned(bias, 16) || !aligned(gamma, 16) ||
      (out && !aligned(out, 8)))
    return OMNI_ERR_INVALID_ARG;
  if (rows == 0) return OMNI_OK;
  ScaleResidualParams p{r, rows, channels, static_cast<const u16*>(y), y_stride, bias, gamma,
                        static_cast<u16*>(out), out_stride};
  hipLaunchKernelGGL(bias_scale_residual_kernel, dim3(blocks_for(rows * (channels / 4), 256)),
                     dim3(256), 0, reinterpret_cast<hipStream_t>(stream), p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_advance_positions(int64_t* positions, int64_t num_slots,
                                      const int64_t* slot_index, int64_t rows,
                                      int64_t new_frames, int cold, omni_stream_t stream) {
  if (!positions || !slot_index || rows < 0 || new_frames < 0) return OMNI_ERR_INVALID_ARG;
  if (rows == 0) return OMNI_OK;
  hipLaunchKernelGGL(advance_positions_kernel, dim3(blocks_for(rows, 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), positions, num_slots, slot_index,
                     rows, new_frames, cold);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}
