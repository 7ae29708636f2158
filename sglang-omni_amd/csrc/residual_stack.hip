// C ABI of the residual-stack kernel: argument validation and the tiling of the position space.
#include "residual_stack.h"

namespace {

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// Compute units of the current device (the sweep sizes its grid to one workgroup per unit),
// queried once per process; 256 (MI355X) when the query fails.
int64_t compute_units() {
  static const int64_t cached = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n < 1) {
      (void)hipGetLastError();
      return (int64_t)256;
    }
    return (int64_t)n;
  }();
  return cached;
}

// The arrays the coefficient rows come from (omni_stack::stack_coef).
void coef_sources(const omni_residual_stack_args* a, bool fp8, omni_stack::StackParams& p) {
  p.nunits = a->num_units;
  for (int k = 0; k < a->num_units; ++k) {
    const omni_residual_unit& u = a->units[k];
    omni_stack::StackUnit& s = p.unit[k];
    s.w1_scale = fp8 ? u.weight1_scale : nullptr;
    s.b1 = u.bias1;
    s.in_a = u.in_act_a;
    s.in_b = u.in_act_b;
    s.mid_a = u.mid_act_a;
    s.mid_b = u.mid_act_b;
    s.w2_scale = fp8 ? u.weight2_scale : nullptr;
    s.b2 = u.bias2;
  }
  p.out_a = a->out_act_a;
  p.out_b = a->out_act_b;
}

}  // namespace

extern "C" int omni_residual_stack_coefficients(const omni_residual_stack_args* a, float* table,
                                                int64_t table_floats, omni_stream_t stream) {
  using namespace omni_stack;
  if (!a || !table || !a->out_act_a || !a->out_act_b) return OMNI_ERR_INVALID_ARG;
  if (a->num_units < 1 || a->num_units > kMaxUnits) return OMNI_ERR_INVALID_ARG;
  if (a->channels != 96) return OMNI_ERR_UNSUPPORTED;
  if (a->weight_dtype != OMNI_DTYPE_BF16 && a->weight_dtype != OMNI_DTYPE_FP8_E4M3)
    return OMNI_ERR_INVALID_ARG;
  const bool fp8 = a->weight_dtype == OMNI_DTYPE_FP8_E4M3;
  for (int k = 0; k < a->num_units; ++k) {
    const omni_residual_unit& u = a->units[k];
    if (!u.in_act_a || !u.in_act_b || !u.mid_act_a || !u.mid_act_b) return OMNI_ERR_INVALID_ARG;
    if (fp8 && (!u.weight1_scale || !u.weight2_scale)) return OMNI_ERR_INVALID_ARG;
  }
  const int n = (a->num_units * kCoefRows + 2) * 96;
  if (table_floats != n || !aligned16(table)) return OMNI_ERR_INVALID_ARG;
  StackParams p{};
  coef_sources(a, fp8, p);
  hipLaunchKernelGGL(stack_coef_kernel<96>, dim3((n + 255) / 256), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), p, table);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_residual_stack(const omni_residual_stack_args* a, omni_stream_t stream) {
  using namespace omni_stack;
  if (!a || !a->x || !a->out_act_a || !a->out_act_b) return OMNI_ERR_INVALID_ARG;
  const bool fin = a->final_weight != nullptr;
  if (!a->out && !fin) return OMNI_ERR_INVALID_ARG;
  if (a->batch < 0 || a->length < 0 || a->num_units < 1 || a->num_units > kMaxUnits)
    return OMNI_ERR_INVALID_ARG;
  if (a->weight_dtype != OMNI_DTYPE_BF16 && a->weight_dtype != OMNI_DTYPE_FP8_E4M3)
    return OMNI_ERR_INVALID_ARG;
  const bool fp8 = a->weight_dtype == OMNI_DTYPE_FP8_E4M3;
  const int64_t C = a->channels;
  if (C != 96) return C > 0 && C % 32 == 0 ? OMNI_ERR_UNSUPPORTED : OMNI_ERR_INVALID_ARG;
  if (a->x_dtype != OMNI_DTYPE_F32 && a->x_dtype != OMNI_DTYPE_F16) return OMNI_ERR_INVALID_ARG;
  const bool x_f16 = a->x_dtype == OMNI_DTYPE_F16;
  const int64_t x_elem = x_f16 ? 2 : 4;
  // 16-byte accesses of out rows; 16-byte (float32) or 8-byte (float16) accesses of x and x_out
  auto x_aligned = [&](const void* ptr) {
    return (reinterpret_cast<uintptr_t>(ptr) & (x_f16 ? 7 : 15)) == 0;
  };
  if (!x_aligned(a->x) || a->x_stride_t < C || a->x_stride_t % 4 || a->x_stride_b % 4)
    return OMNI_ERR_INVALID_ARG;
  if (a->out &&
      (!aligned16(a->out) || a->out_stride_t < C || a->out_stride_t % 8 || a->out_stride_b % 8))
    return OMNI_ERR_INVALID_ARG;
  if (fin) {
    if (!a->final_out || a->final_taps < 1 || a->final_out_stride_b < a->length)
      return OMNI_ERR_INVALID_ARG;
    if (a->final_taps > 8) return OMNI_ERR_UNSUPPORTED;
    if (a->final_activation != OMNI_ACTIVATION_NONE && a->final_activation != OMNI_ACTIVATION_TANH &&
        a->final_activation != OMNI_ACTIVATION_CLAMP)
      return OMNI_ERR_INVALID_ARG;
    if (a->final_hist_pool &&
        (!aligned16(a->final_hist_pool) || a->final_taps < 2 ||
         a->final_hist_slot_stride < 2 * (a->final_taps - 1) * C || a->final_hist_slot_stride % 8))
      return OMNI_ERR_INVALID_ARG;
  }
  if (a->coef_table && !aligned16(a->coef_table)) return OMNI_ERR_INVALID_ARG;
  if (a->x_out && (!x_aligned(a->x_out) || a->x_out_stride_t < C || a->x_out_stride_t % 4 ||
                   a->x_out_stride_b % 4))
    return OMNI_ERR_INVALID_ARG;
  bool any_hist = false;
  int64_t H = 0;
  for (int k = 0; k < a->num_units; ++k) {
    const omni_residual_unit& u = a->units[k];
    if (!u.weight1 || !u.weight2 || !u.in_act_a || !u.in_act_b || !u.mid_act_a || !u.mid_act_b)
      return OMNI_ERR_INVALID_ARG;
    if (!aligned16(u.weight1) || !aligned16(u.weight2)) return OMNI_ERR_INVALID_ARG;
    if (fp8 && (!u.weight1_scale || !u.weight2_scale)) return OMNI_ERR_INVALID_ARG;
    if (u.dilation < 1) return OMNI_ERR_INVALID_ARG;
    if (6 * u.dilation > 60) return OMNI_ERR_UNSUPPORTED;
    if (u.hist_pool) {
      if (!aligned16(u.hist_pool) || u.hist_slot_stride < 2 * 6 * u.dilation * C ||
          u.hist_slot_stride % 8)
        return OMNI_ERR_INVALID_ARG;
      any_hist = true;
    }
    H += 6 * u.dilation;
  }
  if (fin) {
    H += a->final_taps - 1;
    if (a->final_hist_pool) any_hist = true;
  }
  if (any_hist && (!a->slot_index || !a->slot_parity || a->hist_num_slots < 1))
    return OMNI_ERR_INVALID_ARG;
  if (a->batch == 0 || a->length == 0) return OMNI_OK;
  const int64_t R = Stack96Dma::R;  // staged rows per tile (both weight formats)
  if (H + 16 > R) return OMNI_ERR_UNSUPPORTED;

  // byte extents (buffer offsets are 32-bit)
  const int64_t B = a->batch, L = a->length;
  const int64_t limit = 0x7fffffffLL;
  const int64_t x_bytes = ((B - 1) * a->x_stride_b + (L - 1) * a->x_stride_t + C) * x_elem;
  const int64_t o_bytes =
      a->out ? ((B - 1) * a->out_stride_b + (L - 1) * a->out_stride_t + C) * 2 : 0;
  const int64_t fh_bytes =
      fin && a->final_hist_pool ? a->hist_num_slots * a->final_hist_slot_stride * 2 : 0;
  if (fin && ((B - 1) * a->final_out_stride_b + L > limit || fh_bytes > limit))
    return OMNI_ERR_UNSUPPORTED;
  const int64_t xo_bytes =
      a->x_out ? ((B - 1) * a->x_out_stride_b + (L - 1) * a->x_out_stride_t + C) * x_elem : 0;
  if (x_bytes > limit || o_bytes > limit || xo_bytes > limit) return OMNI_ERR_UNSUPPORTED;

  StackParams p{};
  p.x = a->x;
  p.x_f16 = x_f16 ? 1 : 0;
  p.x_sb = (int)a->x_stride_b;
  p.x_st = (int)a->x_stride_t;
  p.batch = (int)B;
  p.length = (int)L;
  p.nunits = a->num_units;
  const int64_t w_elem = fp8 ? 1 : 2;
  for (int k = 0; k < a->num_units; ++k) {
    const omni_residual_unit& u = a->units[k];
    StackUnit& s = p.unit[k];
    s.w1 = u.weight1;
    s.w1_scale = fp8 ? u.weight1_scale : nullptr;
    s.b1 = u.bias1;
    s.in_a = u.in_act_a;
    s.in_b = u.in_act_b;
    s.mid_a = u.mid_act_a;
    s.mid_b = u.mid_act_b;
    s.w2 = u.weight2;
    s.w2_scale = fp8 ? u.weight2_scale : nullptr;
    s.b2 = u.bias2;
    s.dil = (int)u.dilation;
    s.halo = (int)(6 * u.dilation);
    s.w1_bytes = (uint32_t)(C * C * kTaps * w_elem);
    s.w2_bytes = (uint32_t)(C * C * w_elem);
    if (u.hist_pool) {
      const int64_t hb = a->hist_num_slots * u.hist_slot_stride * 2;
      if (hb > limit) return OMNI_ERR_UNSUPPORTED;
      s.hist = reinterpret_cast<u16*>(u.hist_pool);
      s.hist_stride = (int)u.hist_slot_stride;
      s.hist_bytes = (uint32_t)hb;
    }
  }
  p.slot_index = a->slot_index;
  p.slot_parity = a->slot_parity;
  p.hist_slots = a->hist_num_slots;
  p.hist_cold = a->history_cold;
  p.out_a = a->out_act_a;
  p.out_b = a->out_act_b;
  p.out = reinterpret_cast<u16*>(a->out);
  p.o_sb = (int)a->out_stride_b;
  p.o_st = (int)a->out_stride_t;
  p.x_out = a->x_out;
  p.xo_sb = (int)a->x_out_stride_b;
  p.xo_st = (int)a->x_out_stride_t;
  p.x_bytes = (uint32_t)x_bytes;
  p.o_bytes = (uint32_t)o_bytes;
  p.xo_bytes = (uint32_t)xo_bytes;
  p.H = (int)H;
  p.coef_table = a->coef_table;
  if (fin) {
    p.fin_w = a->final_weight;
    p.fin_b = a->final_bias;
    p.fin_taps = (int)a->final_taps;
    p.fin_act = a->final_activation;
    p.fin_hist = reinterpret_cast<u16*>(a->final_hist_pool);
    p.fin_hist_stride = (int)a->final_hist_slot_stride;
    p.fin_hist_bytes = (uint32_t)fh_bytes;
    p.fin_out = a->final_out;
    p.fin_o_sb = a->final_out_stride_b;
  }

  // Long rows: the sweep (each workgroup runs consecutive tiles of one row,
  // the causal halo staged once per workgroup instead of once per tile), one workgroup per
  // compute unit where the rows allow. Otherwise long rows take tiles inside one row, as many as
  // the staged rows need, evened out; short rows as many whole rows (each with its halo) as the
  // staged rows hold.
  int64_t grid;
  bool sweep = false;
  if (L + H > R && a->num_units <= kSweepUnits) {
    int64_t halo_rows = fin ? a->final_taps - 1 : 0;
    bool fits = halo_rows <= kSweepGuard;
    for (int k = 0; k < a->num_units; ++k) {
      halo_rows += 6 * a->units[k].dilation;
      fits = fits && 6 * a->units[k].dilation <= kSweepGuard;
    }
    sweep = fits && halo_rows <= kSweepHaloRows;
  }
  if (sweep) {
    int off = 0;
    for (int k = 0; k <= a->num_units; ++k) {
      const int rows_k = k < a->num_units ? (int)(6 * a->units[k].dilation)
                                          : (fin ? (int)(a->final_taps - 1) : 0);
      p.halo_rows[k] = rows_k;
      p.halo_off[k] = off;
      off += rows_k;
    }
    const int64_t cus = compute_units();
    int64_t segments = B >= cus ? 1 : cus / B;
    // at least two tiles per segment, or the sweep saves no halo
    const int64_t max_segments = (L + 2 * R - 1) / (2 * R);
    segments = segments < 1 ? 1 : (segments > max_segments ? max_segments : segments);
    p.sweep_segments = (int)segments;
    p.sweep_positions = (int)((L + segments - 1) / segments);
    grid = B * segments;
  } else if (L + H > R) {
    const int64_t tiles = (L + (R - H) - 1) / (R - H);
    p.seg_len = (int)((L + tiles - 1) / tiles);
    p.tiles_per_row = (int)((L + p.seg_len - 1) / p.seg_len);
    grid = B * p.tiles_per_row;
  } else {
    p.seg_len = (int)L;
    p.tiles_per_row = 0;
    p.rows_per_tile = (int)(R / (L + H));
    grid = (B + p.rows_per_tile - 1) / p.rows_per_tile;
  }
  if (grid > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return fp8 ? launch_stack96<true>(p, (int)grid, sweep, s)
             : launch_stack96<false>(p, (int)grid, sweep, s);
}
