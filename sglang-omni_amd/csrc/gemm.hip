// The row GEMMs of the code2wav pre-transformer and the ConvNeXt upsamplers (gfx950 bf16 MFMA):
// out = epilogue(A x W^T) with A [rows][k] bf16 and W [n][k] bf16 (a linear layer's weight as
// stored, [out_features][in_features]), float32 accumulation.
//
// Replaces, for the qwen3_omni / qwen3_tts code2wav front ends:
//   F.linear(normed, qkv_weight)                       code2wav.py:267          (STORE)
//   addcmul(residual, scale, F.linear(attended, o))    code2wav.py:311-315      (SCALED_RESIDUAL)
//   silu_and_mul(F.linear(normed, gate_up_weight))     code2wav.py:321          (SILU_MUL)
//   addcmul(hidden, scale, F.linear(activated, down))  code2wav.py:322-326      (SCALED_RESIDUAL)
//   act(pwconv1(normed))                               incremental_codec.py:174-176 (GELU)
//   residual + gamma * pwconv2(...)                    incremental_codec.py:174-180 (SCALED_RESIDUAL)
// (sglang_omni/models/qwen3_omni/components/), so the elementwise passes after each GEMM run in
// its epilogue on the float32 accumulators.
//
// Workgroup: 4 waves (2 x 2) over a tile of BM rows x BN columns, each wave TM x TN MFMA tiles of
// 16 x 16 (v_mfma_f32_16x16x32_bf16). K runs in stages of 64: the stage's A rows and W rows travel
// by LDS DMA (buffer_load ... lds, 16 bytes a lane) into a ring of S stages, S - 1 of them in
// flight while one is multiplied, with one barrier per stage. An LDS row is 64 bf16 (8 slots of 16
// bytes), slot s of row r stored at s ^ (r % 8), so the operand reads of 16 rows spread over all
// banks; each DMA lane loads the global piece that belongs in its slot.
//
// Every output element accumulates its K products in one fixed order (stage by stage, the two
// 32-wide MFMA steps of a stage in order) whatever the tile or the row count, so a row's result
// does not depend on the rows it is batched with: a chunked decode and the whole decode give the
// same bits.
#include "common.h"
#include "omni_codec.h"
#include "rope.h"

namespace {

constexpr int kBK = 64;         // K per stage
constexpr int kRowSlots = 8;    // 16-byte slots per staged row

struct GemmParams {
  const void* a;
  uint32_t a_bytes;
  int a_stride;  // elements
  const void* w;
  uint32_t w_bytes;
  int rows, k, n;
  const float* bias;
  int epi;
  int out_f32;  // SCALED_RESIDUAL: float32 out (else bf16)
  const float* scale;
  const float* res;
  uint32_t res_bytes;
  int res_stride;
  void* out;
  uint32_t out_bytes;
  int out_stride;
  int row_tiles, col_tiles;
  // the rotary epilogue (omni_gemm_rope_kv): rows are batch * frames tokens, out the qkv rows
  int frames, heads, kv_heads;
  const float* inv_freq;
  const int64_t* slot_index;
  const int64_t* positions;
  int cold;
  int64_t num_slots;
  u16* key_ring;
  u16* value_ring;
  int64_t ring_frames;
};

OMNI_DEVICE uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}
OMNI_DEVICE float silu(float g) { return g / (1.f + __expf(-g)); }
OMNI_DEVICE float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }

template <int WM, int WN, int TM, int TN, int S>
struct GemmTile {
  static constexpr int NW = WM * WN;  // waves: WM down the rows, WN across the columns
  static constexpr int BM = WM * TM * 16;
  static constexpr int BN = WN * TN * 16;
  static constexpr int A_ELEMS = BM * kBK;
  static constexpr int B_ELEMS = BN * kBK;
  static constexpr int STAGE = A_ELEMS + B_ELEMS;  // bf16 elements
  static constexpr size_t lds_bytes() { return (size_t)S * STAGE * 2; }
  // 64-lane DMA instructions of a stage (each fills 8 staged rows), shared by the waves
  static constexpr int A_PER_WAVE = BM * kRowSlots / 64 / NW;
  static constexpr int B_PER_WAVE = BN * kRowSlots / 64 / NW;
  static constexpr int PER_WAVE = A_PER_WAVE + B_PER_WAVE;
  static_assert((BM * kRowSlots / 64) % NW == 0 && (BN * kRowSlots / 64) % NW == 0, "DMA split");
};

// The rotary epilogue of the qkv GEMM: a wave's 64 columns are one head (q heads, then k heads,
// then v heads), and lane (g, n) holds columns 16 j + 4 g + e of tile j, so the neox pair (i,
// i + 32) of a q or k head sits in the same lane, in tiles j and j + 2. Each value is rounded to
// bf16 first, as the stored qkv would be, then turned at its token's position and rounded again;
// the rotated k and the v of each token also go to its slot's ring row. What the epilogue reads
// besides the accumulators (the rows' slots, then their positions, inv_freq, the bias) is loaded
// before and during the K loop: at the end it would be two dependent round trips to memory.
template <int TM>
struct RopeRows {
  int64_t slot[TM];  // slot_index of the row's stream (-1: none, or out of range)
  int64_t pos[TM];   // the row's position: its stream's start + its frame
  f32x4 inv[2];      // inv_freq of the lane's pairs 16 j + 4 g + e, j = 0, 1
  f32x4 bias[4];     // the lane's bias of tiles 0 .. 3 (zeros without a bias)
};

// Before the first DMA: the slots, inv_freq and the bias, as buffer loads whose absent operands
// read zeros (no branch around a load: the wait for the slots then covers only these loads).
template <int TM>
OMNI_DEVICE void rope_rows_start(const GemmParams& p, int row0, int c0, int ln, RopeRows<TM>& r) {
  const int g4 = (ln >> 4) * 4;
  const auto srs = buffer_rsrc(p.slot_index, p.slot_index ? (uint32_t)(p.rows / p.frames) * 8u : 0u);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = row0 + i * 16 + (ln & 15);
    const bool ok = row < p.rows && p.slot_index != nullptr;
    const u32x2 w = __builtin_bit_cast(
        u32x2, __builtin_amdgcn_raw_buffer_load_b64(srs, ok ? (uint32_t)(row / p.frames) * 8u : kOutOfRange, 0, 0));
    const int64_t slot = ok ? (int64_t)(((uint64_t)w[1] << 32) | w[0]) : -1;
    r.slot[i] = (slot < 0 || slot >= p.num_slots) ? -1 : slot;
  }
  const auto frs = buffer_rsrc(p.inv_freq, 128u);
  const auto brs = buffer_rsrc(p.bias, p.bias ? (uint32_t)p.n * 4u : 0u);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    r.inv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(frs, (uint32_t)(16 * j + g4) * 4u, 0, 0));
#pragma unroll
  for (int j = 0; j < 4; ++j)
    r.bias[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(brs, (uint32_t)(c0 + 16 * j + g4) * 4u, 0, 0));
}

// After the first DMAs are issued: each row's position (0 for a first decode or no slot).
template <int TM>
OMNI_DEVICE void rope_rows_positions(const GemmParams& p, int row0, int ln, RopeRows<TM>& r) {
  const auto prs = buffer_rsrc(p.positions, p.positions ? (uint32_t)p.num_slots * 8u : 0u);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = row0 + i * 16 + (ln & 15);
    const bool warm = !p.cold && p.positions != nullptr && r.slot[i] >= 0;
    const u32x2 w = __builtin_bit_cast(
        u32x2, __builtin_amdgcn_raw_buffer_load_b64(prs, warm ? (uint32_t)r.slot[i] * 8u : kOutOfRange, 0, 0));
    const int64_t start = warm ? (int64_t)(((uint64_t)w[1] << 32) | w[0]) : 0;
    r.pos[i] = start + (row < p.rows ? row % p.frames : 0);
  }
}

template <int TM>
OMNI_DEVICE void rope_kv_epilogue(const GemmParams& p, const f32x4 (&acc)[TM][4],
                                  const RopeRows<TM>& r, int row0, int c0, int ln,
                                  __amdgpu_buffer_rsrc_t orsrc) {
  const int head = c0 >> 6;
  const int qk_heads = p.heads + p.kv_heads;
  const int kv_width = p.kv_heads * 64;
  const int g4 = (ln >> 4) * 4;
  // acc + bias as the plain store forms it (no add without a bias: -0 stays -0)
  f32x4 v[TM][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i) v[i][j] = p.bias ? acc[i][j] + r.bias[j] : acc[i][j];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = row0 + i * 16 + (ln & 15);
    const bool row_ok = row < p.rows;
    const int64_t pos = r.pos[i];
    const bool ring = row_ok && r.slot[i] >= 0 && p.key_ring != nullptr;
    const int64_t ring_row = ring ? r.slot[i] * p.ring_frames + pos % p.ring_frames : 0;
    if (head < qk_heads) {
      const float fpos = (float)pos;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ci = 16 * j + g4;  // the pair index of element 0
        u16 y1[4], y2[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x1 = bits_to_float_bf16(float_to_bits_bf16(v[i][j][e]));
          const float x2 = bits_to_float_bf16(float_to_bits_bf16(v[i][j + 2][e]));
          rope_pair(x1, x2, fpos * r.inv[j][e], &y1[e], &y2[e]);
        }
        const u32x2 v1 = {(uint32_t)y1[0] | ((uint32_t)y1[1] << 16), (uint32_t)y1[2] | ((uint32_t)y1[3] << 16)};
        const u32x2 v2 = {(uint32_t)y2[0] | ((uint32_t)y2[1] << 16), (uint32_t)y2[2] | ((uint32_t)y2[3] << 16)};
        const uint32_t off = row_ok ? (uint32_t)(row * p.out_stride + c0 + ci) * 2u : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b64(v1, orsrc, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b64(v2, orsrc, row_ok ? off + 64u : kOutOfRange, 0, 0);
        if (ring && head >= p.heads) {
          u16* k = p.key_ring + ring_row * kv_width + (c0 - p.heads * 64) + ci;
          *reinterpret_cast<u32x2*>(k) = v1;
          *reinterpret_cast<u32x2*>(k + 32) = v2;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ci = 16 * j + g4;
        const u32x2 o = {pack_bf16x2(v[i][j][0], v[i][j][1]), pack_bf16x2(v[i][j][2], v[i][j][3])};
        const uint32_t off = row_ok ? (uint32_t)(row * p.out_stride + c0 + ci) * 2u : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b64(o, orsrc, off, 0, 0);
        if (ring)
          *reinterpret_cast<u32x2*>(p.value_ring + ring_row * kv_width + (c0 - qk_heads * 64) + ci) = o;
      }
    }
  }
}

template <int WM, int WN, int TM, int TN, int S, bool ROPE = false>
__global__ void __launch_bounds__(64 * WM * WN) gemm_kernel(const GemmParams p) {
  using T = GemmTile<WM, WN, TM, TN, S>;
  static_assert(!ROPE || TN == 4, "the rotary epilogue takes one 64-column head per wave");
  extern __shared__ __attribute__((aligned(16))) u16 lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM;
  const int wn = wave / WM;
  // tiles column-major (row tiles inner), each XCD a contiguous range: the workgroups of one XCD
  // share W's column blocks in its L2
  const int tile = xcd_tile(blockIdx.x, p.row_tiles * p.col_tiles);
  const int ct = tile / p.row_tiles;
  const int rt = tile - ct * p.row_tiles;
  const int m0 = rt * T::BM;
  const int n0 = ct * T::BN;

  // DMA lane offsets (bytes, the stage's K offset goes in the scalar offset): lane j of
  // instruction i fills slot 64 i + j of the stage region: staged row 8 i + j / 8, physical slot
  // j % 8, which holds logical slot (j % 8) ^ (row % 8)
  const auto ar = buffer_rsrc(p.a, p.a_bytes);
  const auto wr = buffer_rsrc(p.w, p.w_bytes);
  uint32_t a_off[T::A_PER_WAVE], b_off[T::B_PER_WAVE];
  {
    const int ln = opaque_copy(lane);
#pragma unroll
    for (int i = 0; i < T::A_PER_WAVE; ++i) {
      const int row = (wave * T::A_PER_WAVE + i) * 8 + (ln >> 3);
      const int slot = (ln & 7) ^ (row & 7);
      a_off[i] = m0 + row < p.rows ? (uint32_t)((m0 + row) * p.a_stride + slot * 8) * 2u : kOutOfRange;
    }
#pragma unroll
    for (int i = 0; i < T::B_PER_WAVE; ++i) {
      const int row = (wave * T::B_PER_WAVE + i) * 8 + (ln >> 3);
      const int slot = (ln & 7) ^ (row & 7);
      b_off[i] = n0 + row < p.n ? (uint32_t)((n0 + row) * p.k + slot * 8) * 2u : kOutOfRange;
    }
  }
  const int stages = p.k / kBK;
  auto issue = [&](int kt) __attribute__((always_inline)) {
    u16* st = lds + (kt % S) * T::STAGE;
    const int kb = kt * kBK * 2;
#pragma unroll
    for (int i = 0; i < T::A_PER_WAVE; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ar, (__attribute__((address_space(3))) void*)(st + (wave * T::A_PER_WAVE + i) * 512), 16,
          (int)a_off[i], kb, 0, 0);
#pragma unroll
    for (int i = 0; i < T::B_PER_WAVE; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wr, (__attribute__((address_space(3))) void*)(st + T::A_ELEMS +
                                                        (wave * T::B_PER_WAVE + i) * 512),
          16, (int)b_off[i], kb, 0, 0);
  };

  // operand reads: row r (a multiple of 16 plus lane % 16) of the A or W region, logical slot
  // 4 s + lane / 16 for MFMA step s of the stage
  const int lr = lane & 15;
  const int lq = lane >> 4;
  const int rd0 = ((lq) ^ (lr & 7)) * 8 + lr * kBK;
  const int rd1 = ((4 + lq) ^ (lr & 7)) * 8 + lr * kBK;
  const int a_base = wm * TM * 16 * kBK;
  const int b_base = T::A_ELEMS + wn * TN * 16 * kBK;

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  RopeRows<ROPE ? TM : 1> rope;
  if constexpr (ROPE) rope_rows_start<TM>(p, m0 + wm * TM * 16, n0 + wn * TN * 16, lane, rope);
#pragma unroll
  for (int kt = 0; kt < S - 1; ++kt)
    if (kt < stages) issue(kt);
  if constexpr (ROPE) rope_rows_positions<TM>(p, m0 + wm * TM * 16, lane, rope);
  for (int kt = 0; kt < stages; ++kt) {
    // this wave's DMA of stage kt is complete once at most the later stages' instructions are
    // outstanding; then every wave's (the barrier), which also ends every read of the buffer that
    // stage kt + S - 1 refills
    if (kt + S - 2 < stages) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 2) * T::PER_WAVE) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("s_barrier" ::: "memory");
    if (kt + S - 1 < stages) issue(kt + S - 1);
    const u16* st = lds + (kt % S) * T::STAGE;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int rd = s ? rd1 : rd0;
      bf16x8 av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        av[i] = *reinterpret_cast<const bf16x8*>(st + a_base + i * 16 * kBK + rd);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bv[j] = *reinterpret_cast<const bf16x8*>(st + b_base + j * 16 * kBK + rd);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bv[j], av[i], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue: lane holds row m0 + wm TM 16 + 16 i + lane % 16, columns n0 + wn TN 16 + 16 j +
  // 4 (lane / 16) .. + 3 of tile (i, j)
  const auto orsrc = buffer_rsrc(p.out, p.out_bytes);
  const int ln = opaque_copy(lane);
  if constexpr (ROPE) {
    rope_kv_epilogue<TM>(p, acc, rope, m0 + wm * TM * 16, n0 + wn * TN * 16, ln, orsrc);
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = m0 + wm * TM * 16 + i * 16 + (ln & 15);
    const bool row_ok = row < p.rows;
    if (TN % 2 == 0 && p.epi == OMNI_GEMM_SILU_MUL) {
      // W's rows interleaved by 16: column block 2 q gates, 2 q + 1 ups of output columns
      // 16 q .. 16 q + 15
#pragma unroll
      for (int j = 0; j + 1 < TN; j += 2) {
        const int col = n0 + wn * TN * 16 + j * 16 + (ln >> 4) * 4;
        const int oc = (col >> 5) * 16 + (col & 15);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float g = acc[i][j][e] + (p.bias ? p.bias[col + e] : 0.f);
          const float u = acc[i][j + 1][e] + (p.bias ? p.bias[col + 16 + e] : 0.f);
          o[e] = silu(g) * u;
        }
        const bool ok = row_ok && col < p.n;
        const uint32_t off = ok ? (uint32_t)(row * p.out_stride + oc) * 2u : kOutOfRange;
        const u32x2 v = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        __builtin_amdgcn_raw_buffer_store_b64(v, orsrc, off, 0, 0);
      }
      continue;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * TN * 16 + j * 16 + (ln >> 4) * 4;
      const bool ok = row_ok && col < p.n;
      f32x4 v = acc[i][j];
      if (p.bias) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(p.bias + (col < p.n ? col : 0));
        v += b;
      }
      if (p.epi == OMNI_GEMM_SCALED_RESIDUAL) {
        const auto rr = buffer_rsrc(p.res, p.res_bytes);
        const uint32_t roff = ok ? (uint32_t)(row * p.res_stride + col) * 4u : kOutOfRange;
        const f32x4 r = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, roff, 0, 0));
        const f32x4 sc = *reinterpret_cast<const f32x4*>(p.scale + (col < p.n ? col : 0));
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(sc[e], v[e], r[e]);
        if (p.out_f32) {
          const uint32_t off = ok ? (uint32_t)(row * p.out_stride + col) * 4u : kOutOfRange;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), orsrc, off, 0, 0);
        } else {
          const uint32_t off = ok ? (uint32_t)(row * p.out_stride + col) * 2u : kOutOfRange;
          const u32x2 ob = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
          __builtin_amdgcn_raw_buffer_store_b64(ob, orsrc, off, 0, 0);
        }
      } else {
        if (p.epi == OMNI_GEMM_GELU) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = gelu_erf(v[e]);
        }
        const uint32_t off = ok ? (uint32_t)(row * p.out_stride + col) * 2u : kOutOfRange;
        const u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        __builtin_amdgcn_raw_buffer_store_b64(o, orsrc, off, 0, 0);
      }
    }
  }
}

template <int WM, int WN, int TM, int TN, int S, bool ROPE = false>
int launch(GemmParams p, hipStream_t stream) {
  using T = GemmTile<WM, WN, TM, TN, S>;
  p.row_tiles = (p.rows + T::BM - 1) / T::BM;
  p.col_tiles = (p.n + T::BN - 1) / T::BN;
  auto k = gemm_kernel<WM, WN, TM, TN, S, ROPE>;
  static const bool raised = [&] {
    return hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)T::lds_bytes()) == hipSuccess;
  }();
  if (!raised) return OMNI_ERR_LAUNCH;
  hipLaunchKernelGGL(k, dim3((unsigned)(p.row_tiles * p.col_tiles)), dim3(64 * T::NW), T::lds_bytes(),
                     stream, p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

int64_t tiles_of(int64_t rows, int64_t n, int bm, int bn) {
  return ((rows + bm - 1) / bm) * ((n + bn - 1) / bn);
}

int compute_units() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 256;
  return cus;
}

bool aligned_to(const void* ptr, int bytes) {
  return (reinterpret_cast<uintptr_t>(ptr) & (uintptr_t)(bytes - 1)) == 0;
}

// The checks and kernel parameters shared by the entry points; kNothingToDo (with *out
// untouched): rows = 0.
constexpr int kNothingToDo = -1;  // no OMNI_ERR_* code
int gemm_params(const omni_gemm_args* a, GemmParams* out) {
  if (a == nullptr || a->a == nullptr || a->w == nullptr || a->out == nullptr)
    return OMNI_ERR_INVALID_ARG;
  if (a->rows < 0 || a->k <= 0 || a->n <= 0 || a->k % kBK != 0 || a->n % 64 != 0)
    return OMNI_ERR_INVALID_ARG;
  if (a->rows == 0) return kNothingToDo;
  const int epi = a->epilogue;
  if (epi != OMNI_GEMM_STORE && epi != OMNI_GEMM_SILU_MUL && epi != OMNI_GEMM_GELU &&
      epi != OMNI_GEMM_SCALED_RESIDUAL)
    return OMNI_ERR_INVALID_ARG;
  if (epi == OMNI_GEMM_SCALED_RESIDUAL && (a->scale == nullptr || a->residual == nullptr))
    return OMNI_ERR_INVALID_ARG;
  const int64_t out_cols = epi == OMNI_GEMM_SILU_MUL ? a->n / 2 : a->n;
  // float32 out only for the scaled residual
  if (a->out_dtype != OMNI_DTYPE_BF16 &&
      !(a->out_dtype == OMNI_DTYPE_F32 && epi == OMNI_GEMM_SCALED_RESIDUAL))
    return OMNI_ERR_INVALID_ARG;
  const bool out_f32 = a->out_dtype == OMNI_DTYPE_F32;
  if (a->a_stride < a->k || a->out_stride < out_cols ||
      (epi == OMNI_GEMM_SCALED_RESIDUAL && a->residual_stride < a->n))
    return OMNI_ERR_INVALID_ARG;
  // 16-byte operand rows, 8-byte (bf16) or 16-byte (float32) output pieces
  const int ob = out_f32 ? 4 : 2;
  if (!aligned_to(a->a, 16) || (a->a_stride * 2) % 16 != 0 || !aligned_to(a->w, 16) ||
      !aligned_to(a->out, 4 * ob) || (a->out_stride * ob) % (4 * ob) != 0 ||
      (a->bias != nullptr && !aligned_to(a->bias, 16)))
    return OMNI_ERR_INVALID_ARG;
  if (epi == OMNI_GEMM_SCALED_RESIDUAL &&
      (!aligned_to(a->residual, 16) || (a->residual_stride * 4) % 16 != 0 ||
       !aligned_to(a->scale, 16)))
    return OMNI_ERR_INVALID_ARG;
  const int64_t a_bytes = ((a->rows - 1) * a->a_stride + a->k) * 2;
  const int64_t w_bytes = a->n * a->k * 2;
  const int64_t o_bytes = ((a->rows - 1) * a->out_stride + out_cols) * ob;
  const int64_t r_bytes =
      epi == OMNI_GEMM_SCALED_RESIDUAL ? ((a->rows - 1) * a->residual_stride + a->n) * 4 : 0;
  const int64_t limit = 0x7fffffffLL;
  if (a_bytes >= limit || w_bytes >= limit || o_bytes >= limit || r_bytes >= limit)
    return OMNI_ERR_UNSUPPORTED;
  GemmParams& p = *out;
  p = GemmParams{};
  p.a = a->a;
  p.a_bytes = (uint32_t)a_bytes;
  p.a_stride = (int)a->a_stride;
  p.w = a->w;
  p.w_bytes = (uint32_t)w_bytes;
  p.rows = (int)a->rows;
  p.k = (int)a->k;
  p.n = (int)a->n;
  p.bias = a->bias;
  p.epi = epi;
  p.out_f32 = out_f32 ? 1 : 0;
  p.scale = a->scale;
  p.res = a->residual;
  p.res_bytes = (uint32_t)r_bytes;
  p.res_stride = (int)a->residual_stride;
  p.out = a->out;
  p.out_bytes = (uint32_t)o_bytes;
  p.out_stride = (int)a->out_stride;
  return OMNI_OK;
}

}  // namespace

extern "C" int omni_gemm(const omni_gemm_args* a, omni_stream_t stream) {
  GemmParams p;
  const int rc = gemm_params(a, &p);
  if (rc != OMNI_OK) return rc == kNothingToDo ? OMNI_OK : rc;
  const int epi = a->epilogue;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // The tiles (rows x columns: waves, ring stages, LDS): 1: 64 x 128: 4, 3, 72 KiB; 2: 64 x 64:
  // 4, 4, 64 KiB; 3: 64 x 128: 8 (2 x 4), 3, 72 KiB; 4: 64 x 64: 8 (2 x 4), 4, 64 KiB; 5: 32 x
  // 64: 4, 3, 36 KiB; 6: 64 x 128: 8 (4 x 2), 3, 72 KiB. The automatic choice: 64 x 128 of 8
  // waves where it gives a workgroup per CU, else 64 x 64 of 8 waves (32 x 64 with the gated
  // epilogue, which needs two column tiles per wave). Measured at 768 - 3 072 rows: a second
  // wave per SIMD hides the stage barrier and the LDS latency the one-wave tiles wait on (qkv
  // 768 x 1024 -> 3072 14.4 -> 13.1 us, down 768 x 3072 -> 1024 17.8 -> 16.5 us); deeper rings
  // and 128 x 128 tiles were slower.
  int config = a->config;
  if (config == 0) {
    if (a->n % 128 == 0 && tiles_of(a->rows, a->n, 64, 128) >= compute_units())
      config = 3;
    else
      config = epi == OMNI_GEMM_SILU_MUL ? 5 : 4;
  }
  const int bn = (config == 1 || config == 3 || config == 6) ? 128 : 64;
  if (config >= 1 && config <= 6 && a->n % bn != 0) return OMNI_ERR_UNSUPPORTED;
  if (config == 4 && epi == OMNI_GEMM_SILU_MUL) return OMNI_ERR_UNSUPPORTED;  // one column tile
  switch (config) {
    case 1: return launch<2, 2, 2, 4, 3>(p, s);
    case 2: return launch<2, 2, 2, 2, 4>(p, s);
    case 3: return launch<2, 4, 2, 2, 3>(p, s);
    case 4: return launch<2, 4, 2, 1, 4>(p, s);
    case 5: return launch<2, 2, 1, 2, 3>(p, s);
    case 6: return launch<4, 2, 1, 4, 3>(p, s);
    default: break;
  }
  return OMNI_ERR_INVALID_ARG;
}

extern "C" int omni_gemm_rope_kv(const omni_gemm_args* a, int64_t frames, int64_t heads,
                                 int64_t kv_heads, int64_t head_dim, const float* inv_freq,
                                 const int64_t* slot_index, const int64_t* positions, int cold,
                                 int64_t num_slots, void* key_ring, void* value_ring,
                                 int64_t ring_frames, omni_stream_t stream) {
  // the checks of omni_rope_kv_write, and a plain bf16 store of exactly the q, k, v columns
  if (a == nullptr || a->epilogue != OMNI_GEMM_STORE || a->out_dtype != OMNI_DTYPE_BF16)
    return OMNI_ERR_INVALID_ARG;
  if (!inv_freq || frames < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads)
    return OMNI_ERR_INVALID_ARG;
  if (head_dim != 64) return OMNI_ERR_UNSUPPORTED;
  if (a->n != (heads + 2 * kv_heads) * head_dim || a->rows % frames) return OMNI_ERR_INVALID_ARG;
  if ((key_ring != nullptr) != (value_ring != nullptr)) return OMNI_ERR_INVALID_ARG;
  if (key_ring && (!slot_index || ring_frames < 1)) return OMNI_ERR_INVALID_ARG;
  if (!cold && (!slot_index || !positions)) return OMNI_ERR_INVALID_ARG;
  GemmParams p;
  const int rc = gemm_params(a, &p);
  if (rc != OMNI_OK) return rc == kNothingToDo ? OMNI_OK : rc;
  p.frames = (int)frames;
  p.heads = (int)heads;
  p.kv_heads = (int)kv_heads;
  p.inv_freq = inv_freq;
  p.slot_index = slot_index;
  p.positions = positions;
  p.cold = cold ? 1 : 0;
  p.num_slots = num_slots;
  p.key_ring = static_cast<u16*>(key_ring);
  p.value_ring = static_cast<u16*>(value_ring);
  p.ring_frames = ring_frames;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // one 64-column head per wave: 64 x 128 tiles of 4 waves (2 x 2, each 32 rows) or of 8 (4 x
  // 2, each 16 rows). At 768 x 1024 -> 3072 with rings: 15.3 and 16.1 us (the two-launch form
  // 19.5 us; its GEMM alone 11.1 - 12.1 us, the ring writes ~2.2 us of the difference)
  const int config = a->config == 0 ? 1 : a->config;
  if (a->n % 128 != 0) return OMNI_ERR_UNSUPPORTED;
  switch (config) {
    case 1: return launch<2, 2, 2, 4, 3, true>(p, s);
    case 6: return launch<4, 2, 1, 4, 3, true>(p, s);
    default: break;
  }
  return OMNI_ERR_UNSUPPORTED;
}
