// C ABI of the fused convolution: argument validation and the choice of kernel configuration.
// The kernel template and its tile configurations are in conv_kernel.h.
#include <mutex>

#include "conv_dma.h"
#include "conv_kernel.h"

// The split-K partials of omni_conv1d_splitk_noalloc: one array per GPU (each device holds its own
// copy at its own address), kept until the process ends. In host code `scratch` names a host-side
// stand-in, never the device memory: kernels and copies take the address scratch_address()
// looked up with hipGetSymbolAddress.
constexpr int64_t kScratchBytes = OMNI_SPLITK_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kScratchBytes / 4];

namespace omni_conv {
namespace {

// The kernel family and configuration for p: OMNI_CONV_KERNEL_AUTO picks the family by the
// operand mode, weight dtype and taps (LDS-DMA for bf16 operands used as they are, with bf16 or
// E4M3 weights, then the register-staged kernels) and the configuration by size; a named family
// runs only if it can serve p. `kernel` returns the family that took the call.
int dispatch(const ConvParams& p, bool x_f32, bool fp8, bool fuse2, int& kernel, Choice& ch,
             hipStream_t stream) {
  if (p.halo > kMaxHalo) return OMNI_ERR_UNSUPPORTED;
  const int in_mode = x_f32 ? IN_F32 : (p.in_act != OMNI_ACT_NONE ? IN_ACT : IN_RAW);
  const int want = kernel;
  auto allowed = [&](int family) { return want == OMNI_CONV_KERNEL_AUTO || want == family; };
  if (allowed(OMNI_CONV_KERNEL_DMA) && in_mode == IN_RAW && !fuse2 && p.c_in % kChunk == 0) {
    int status = OMNI_ERR_UNSUPPORTED;
    if (p.taps == 7) status = launch_dma_taps7(p, fp8, ch, stream);
    else if (p.taps == 2) status = launch_dma_taps2(p, fp8, ch, stream);
    else if (p.taps == 1) status = launch_dma_taps1(p, fp8, ch, stream);
    else if (p.taps == 3) status = launch_dma_taps3(p, fp8, ch, stream);
    else if (p.taps == 11) status = launch_dma_taps11(p, fp8, ch, stream);
    if (status != OMNI_ERR_UNSUPPORTED || want == OMNI_CONV_KERNEL_DMA) {
      kernel = OMNI_CONV_KERNEL_DMA;
      return status;
    }
  }
  if (want == OMNI_CONV_KERNEL_DMA) return OMNI_ERR_UNSUPPORTED;
  if (fuse2) {
    if (!allowed(OMNI_CONV_KERNEL_FUSED_UNIT)) return OMNI_ERR_UNSUPPORTED;
    kernel = OMNI_CONV_KERNEL_FUSED_UNIT;
    return fp8 ? launch_fused<true>(p, in_mode, ch, stream)
               : launch_fused<false>(p, in_mode, ch, stream);
  }
  if (p.taps <= 7 && allowed(OMNI_CONV_KERNEL_STAGED)) {
    kernel = OMNI_CONV_KERNEL_STAGED;
    switch (in_mode) {
      case IN_RAW: return fp8 ? launch_taps7<IN_RAW, true>(p, ch, stream) : launch_taps7<IN_RAW, false>(p, ch, stream);
      case IN_ACT: return fp8 ? launch_taps7<IN_ACT, true>(p, ch, stream) : launch_taps7<IN_ACT, false>(p, ch, stream);
      default: return fp8 ? launch_taps7<IN_F32, true>(p, ch, stream) : launch_taps7<IN_F32, false>(p, ch, stream);
    }
  }
  if (p.taps <= 11 && !fp8 && allowed(OMNI_CONV_KERNEL_STAGED11)) {
    kernel = OMNI_CONV_KERNEL_STAGED11;
    return launch_taps11(p, in_mode, ch, stream);
  }
  return OMNI_ERR_UNSUPPORTED;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

bool valid_act(int act, const float* a, const float* b) {
  if (act < OMNI_ACTIVATION_NONE || act > OMNI_ACTIVATION_CLAMP) return false;
  return act != OMNI_ACTIVATION_SNAKE || (a && b);
}

}  // namespace
}  // namespace omni_conv

namespace omni_conv {

// Validates the C-ABI arguments and fills the kernel parameters; OMNI_OK when there is work to
// launch, OMNI_ERR_* on a contract violation, and -1 when the call is valid but empty.
int make_conv_params(const omni_conv_args* a, ConvParams& p, bool& x_f32, bool& fp8, bool& fuse2) {
  if (!a || !a->x || !a->weight) return OMNI_ERR_INVALID_ARG;
  if (!a->out && !a->sum_out) return OMNI_ERR_INVALID_ARG;
  if (a->batch < 0 || a->length < 0 || a->c_in < 1 || a->n_cols < 1 || a->c_out < 1 ||
      a->taps < 1 || a->dilation < 1 || a->left_pad < 0)
    return OMNI_ERR_INVALID_ARG;
  if (a->n_cols % 16 || a->n_cols % a->c_out || a->c_out % 4 || a->c_in % 8)
    return OMNI_ERR_UNSUPPORTED;
  if (a->left_pad > (a->taps - 1) * a->dilation) return OMNI_ERR_INVALID_ARG;
  if (a->x_dtype != OMNI_DTYPE_BF16 && a->x_dtype != OMNI_DTYPE_F32) return OMNI_ERR_INVALID_ARG;
  x_f32 = a->x_dtype == OMNI_DTYPE_F32;
  if (a->in_activation != OMNI_ACTIVATION_NONE && a->in_activation != OMNI_ACTIVATION_SNAKE &&
      a->in_activation != OMNI_ACTIVATION_LEAKY_RELU)
    return OMNI_ERR_INVALID_ARG;
  if (!valid_act(a->in_activation, a->in_act_a, a->in_act_b)) return OMNI_ERR_INVALID_ARG;
  if (a->in_activation == OMNI_ACTIVATION_SNAKE &&
      (!aligned16(a->in_act_a) || !aligned16(a->in_act_b)))
    return OMNI_ERR_INVALID_ARG;
  if (a->weight_dtype != OMNI_DTYPE_BF16 && a->weight_dtype != OMNI_DTYPE_FP8_E4M3)
    return OMNI_ERR_INVALID_ARG;
  fp8 = a->weight_dtype == OMNI_DTYPE_FP8_E4M3;
  if (fp8 && !a->weight_scale) return OMNI_ERR_INVALID_ARG;
  fuse2 = a->weight2 != nullptr;
  if (fuse2) {
    if (a->n_cols != a->c_out || (fp8 && !a->weight2_scale) || !aligned16(a->weight2))
      return OMNI_ERR_INVALID_ARG;
    if (!valid_act(a->mid_activation, a->mid_act_a, a->mid_act_b)) return OMNI_ERR_INVALID_ARG;
  }
  if (a->out_dtype != OMNI_DTYPE_BF16 && a->out_dtype != OMNI_DTYPE_F32)
    return OMNI_ERR_INVALID_ARG;
  if (!valid_act(a->activation, a->act_a, a->act_b)) return OMNI_ERR_INVALID_ARG;
  // 16-byte staging loads of x and history, 16/8-byte epilogue accesses.
  if (!aligned16(a->x) || a->x_stride_t % 8 || a->x_stride_b % 8 || a->x_stride_t < a->c_in)
    return OMNI_ERR_INVALID_ARG;
  if (!aligned16(a->weight)) return OMNI_ERR_INVALID_ARG;
  if (a->x_length < 0) return OMNI_ERR_INVALID_ARG;
  const bool has_r = a->residual || a->sum_out || a->mix_a;
  if (a->residual_dtype != OMNI_DTYPE_F32 && a->residual_dtype != OMNI_DTYPE_F16)
    return OMNI_ERR_INVALID_ARG;
  const bool r_f16 = a->residual_dtype == OMNI_DTYPE_F16;
  if (has_r && (a->residual_stride_t % 4 || a->residual_stride_b % 4 ||
                a->residual_stride_t < a->n_cols))
    return OMNI_ERR_INVALID_ARG;
  // 16-byte float32 / 8-byte float16 accesses of 4 elements
  auto r_aligned = [&](const void* ptr) {
    return (reinterpret_cast<uintptr_t>(ptr) & (r_f16 ? 7 : 15)) == 0;
  };
  if ((a->residual && !r_aligned(a->residual)) || (a->sum_out && !r_aligned(a->sum_out)))
    return OMNI_ERR_INVALID_ARG;
  if (a->mix_a && (!a->mix_b || !r_aligned(a->mix_a) || !r_aligned(a->mix_b)))
    return OMNI_ERR_INVALID_ARG;
  if (a->out && a->out_stride_t < a->n_cols) return OMNI_ERR_INVALID_ARG;
  if (a->out) {
    if ((reinterpret_cast<uintptr_t>(a->out) & 7) || a->out_stride_t % 4 || a->out_stride_b % 4)
      return OMNI_ERR_INVALID_ARG;
    if (a->out_dtype == OMNI_DTYPE_F32 && !aligned16(a->out)) return OMNI_ERR_INVALID_ARG;
  }
  if (a->hist_pool) {
    if (!a->slot_index || !a->slot_parity || !aligned16(a->hist_pool) || a->hist_num_slots < 1)
      return OMNI_ERR_INVALID_ARG;
    if (a->left_pad != (a->taps - 1) * a->dilation) return OMNI_ERR_INVALID_ARG;
    if (a->x_length != 0 && a->x_length != a->length) return OMNI_ERR_INVALID_ARG;
    if (a->hist_slot_stride < 2 * a->left_pad * a->c_in || a->hist_slot_stride % 8)
      return OMNI_ERR_INVALID_ARG;
  }
  if (a->batch == 0 || a->length == 0) return -1;
  const int64_t x_length = a->x_length ? a->x_length : a->length;
  // byte extents of every buffer the kernel touches; buffer offsets are 32-bit
  const int64_t x_elem = x_f32 ? 4 : 2, w_elem = fp8 ? 1 : 2;
  const int64_t chunks = (a->c_in + 31) / 32;
  const int64_t x_bytes =
      ((a->batch - 1) * a->x_stride_b + (x_length - 1) * a->x_stride_t + a->c_in) * x_elem;
  const int64_t w_bytes = chunks * a->n_cols * a->taps * 32 * w_elem;
  const int64_t w2_bytes = fuse2 ? (a->n_cols / 32) * a->n_cols * 32 * w_elem : 0;
  const int64_t hist_bytes = a->hist_pool ? a->hist_num_slots * a->hist_slot_stride * 2 : 0;
  const int64_t r_bytes =
      has_r ? ((a->batch - 1) * a->residual_stride_b + (a->length - 1) * a->residual_stride_t +
               a->n_cols) * (r_f16 ? 2 : 4) : 0;
  const int64_t o_bytes =
      a->out ? ((a->batch - 1) * a->out_stride_b + (a->length - 1) * a->out_stride_t + a->n_cols) *
                   (a->out_dtype == OMNI_DTYPE_F32 ? 4 : 2) : 0;
  const int64_t limit = 0x7fffffffLL;
  if (x_bytes > limit || w_bytes > limit || w2_bytes > limit || hist_bytes > limit ||
      r_bytes > limit || o_bytes > limit)
    return OMNI_ERR_UNSUPPORTED;
  if (fuse2 && a->n_cols % 32) return OMNI_ERR_UNSUPPORTED;
  // in-kernel offsets are 32-bit: positions, x and history element offsets, a chunk of weights
  // (the epilogue splits a flattened position m into (row, position) with a float32 reciprocal
  // of length and a one-step correction, exact while m / length < 2^20)
  if (a->batch > (1 << 20)) return OMNI_ERR_UNSUPPORTED;
  if (a->batch * a->length > 0x3fffffffLL || a->batch * a->x_stride_b > 0x7fffffffLL ||
      (x_length + a->left_pad) * a->x_stride_t > 0x7fffffffLL ||
      a->n_cols * a->taps * 32 > 0x7fffffffLL ||
      (a->hist_pool && a->hist_num_slots * a->hist_slot_stride > 0x7fffffffLL))
    return OMNI_ERR_UNSUPPORTED;

  p = ConvParams{};
  p.x = a->x;
  p.x_sb = a->x_stride_b;
  p.x_st = a->x_stride_t;
  p.batch = (int)a->batch;
  p.length = (int)a->length;
  p.c_in = (int)a->c_in;
  p.x_length = (int)x_length;
  p.in_act = a->in_activation;
  p.in_a = a->in_act_a;
  p.in_b = a->in_act_b;
  p.in_slope = a->in_act_slope;
  p.weight = a->weight;
  p.wscale = fp8 ? a->weight_scale : nullptr;
  p.n_cols = (int)a->n_cols;
  p.c_out = (int)a->c_out;
  p.taps = (int)a->taps;
  p.dil = (int)a->dilation;
  p.lpad = (int)a->left_pad;
  p.halo = (int)((a->taps - 1) * a->dilation);
  p.bias = a->bias;
  p.weight2 = a->weight2;
  p.wscale2 = fp8 ? a->weight2_scale : nullptr;
  p.bias2 = a->bias2;
  p.mid_act = a->mid_activation;
  p.mid_a = a->mid_act_a;
  p.mid_b = a->mid_act_b;
  p.mid_slope = a->mid_act_slope;
  p.hist = reinterpret_cast<const u16*>(a->hist_pool);
  p.slot_index = a->slot_index;
  p.slot_parity = a->slot_parity;
  p.hist_slots = a->hist_num_slots;
  p.hist_slot_stride = a->hist_slot_stride;
  p.hist_cold = a->history_cold;
  p.residual = a->residual;
  p.r_sb = a->residual_stride_b;
  p.r_st = a->residual_stride_t;
  p.mix_a = a->mix_a;
  p.mix_b = a->mix_b;
  p.mix_scale = a->mix_scale;
  p.sum_out = a->sum_out;
  p.r_f16 = r_f16 ? 1 : 0;
  p.out = a->out;
  p.out_bf16 = a->out_dtype == OMNI_DTYPE_BF16;
  p.o_sb = a->out_stride_b;
  p.o_st = a->out_stride_t;
  p.act = a->activation;
  p.act_a = a->act_a;
  p.act_b = a->act_b;
  p.slope = a->act_slope;
  p.x_bytes = (uint32_t)x_bytes;
  p.w_bytes = (uint32_t)w_bytes;
  p.w2_bytes = (uint32_t)w2_bytes;
  p.hist_bytes = (uint32_t)hist_bytes;
  p.r_bytes = (uint32_t)r_bytes;
  p.o_bytes = (uint32_t)o_bytes;
  p.k_splits = 1;
  p.partial = nullptr;
  return OMNI_OK;
}

// The split-K reduction: out[m][n] = act((sum over slices s = 0, 1, .. of partial[s][m][n], in
// slice order) * scale[n] + bias[n % c_out]), the activation (none, Snake with per-channel
// act_a / act_b, LeakyReLU) and the store (bf16 rounded to nearest even, or float32) as the conv
// epilogue applies them. One thread per 4 columns of one position.
// SPLITS > 0 fixes the slice count: every slice's partial is loaded before the first add (in a
// loop each add waited for its load); SPLITS = 0 reads it from `splits`. Slices add in order.
template <int SPLITS>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(
    const float* partial, int splits, int64_t slice, int n_cols, int c_out, int length,
    int quads, const float* scale, const float* bias, int act, const float* act_a,
    const float* act_b, float slope, void* out, int out_bf16, int64_t o_sb, int64_t o_st) {
  const int e = blockIdx.x * 256 + threadIdx.x;  // a slice holds below 2^31 bytes
  if (e >= quads) return;
  const int nq = n_cols / 4;
  const int m = e / nq;
  const int n = (e - m * nq) * 4;
  const float* src = partial + (int64_t)m * n_cols + n;
  f32x4 v;
  if constexpr (SPLITS > 0) {
    f32x4 part[SPLITS];
#pragma unroll
    for (int s = 0; s < SPLITS; ++s) part[s] = *reinterpret_cast<const f32x4*>(src + s * slice);
    v = part[0];
#pragma unroll
    for (int s = 1; s < SPLITS; ++s) v += part[s];
  } else {
    v = *reinterpret_cast<const f32x4*>(src);
    for (int s = 1; s < splits; ++s) v += *reinterpret_cast<const f32x4*>(src + s * slice);
  }
  f32x4 sc = f32x4{1.f, 1.f, 1.f, 1.f}, bi = f32x4{0.f, 0.f, 0.f, 0.f};
  if (scale) sc = *reinterpret_cast<const f32x4*>(scale + n);
  if (bias) {
    const int co = n % c_out;  // c_out is a multiple of 4: the 4 columns share a phase
    bi = f32x4{bias[co], bias[co + 1], bias[co + 2], bias[co + 3]};
  }
  v = v * sc + bi;
  if (act == OMNI_ACT_SNAKE) {
    const int co = n % c_out;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = snake_rev(v[e], act_a[co + e] * kInvTwoPi, act_b[co + e]);
  } else if (act == OMNI_ACT_LEAKY_RELU) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = v[e] >= 0.f ? v[e] : v[e] * slope;
  }
  const int b = m / length;
  const int64_t off = b * o_sb + (int64_t)(m - b * length) * o_st + n;
  if (out_bf16) {
    *reinterpret_cast<u32x2*>(static_cast<u16*>(out) + off) =
        u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + off) = v;
  }
}

}  // namespace omni_conv

namespace {

// Validate, then choose (and launch unless `launch` is false) through dispatch. k_splits > 1: the
// split-K form (see omni_conv1d_splitk) with its float32 partials in `workspace`.
int conv_entry(const omni_conv_args* a, int kernel, int config, bool launch, int* kernel_out,
               int* config_out, int* count_out, int64_t* workgroups_out, omni_stream_t stream,
               int64_t k_splits = 1, float* workspace = nullptr, int64_t workspace_bytes = 0) {
  using namespace omni_conv;
  if (kernel < OMNI_CONV_KERNEL_AUTO || kernel > OMNI_CONV_KERNEL_FUSED_UNIT || config < 0 ||
      (kernel == OMNI_CONV_KERNEL_AUTO && config != 0) || k_splits < 1)
    return OMNI_ERR_INVALID_ARG;
  ConvParams p;
  bool x_f32 = false, fp8 = false, fuse2 = false;
  const int status = make_conv_params(a, p, x_f32, fp8, fuse2);
  if (status != OMNI_OK) {
    if (status < 0 && kernel_out) *kernel_out = OMNI_CONV_KERNEL_AUTO;  // nothing to launch
    return status < 0 ? OMNI_OK : status;
  }
  const int64_t positions = a->batch * a->length;
  if (k_splits > 1) {
    // a k = 1 or k = 7 conv of a bf16 operand (its history rows staged per slice) with bf16
    // weights; bias and an output activation (none, Snake, LeakyReLU) in the reduction; no
    // residual, mix or float32 sum; whole chunks per slice
    if ((a->taps != 1 && a->taps != 7) || fp8 || fuse2 || x_f32 ||
        a->in_activation != OMNI_ACTIVATION_NONE || a->residual || a->mix_a || a->sum_out ||
        !a->out || (p.act != OMNI_ACT_NONE && p.act != OMNI_ACT_SNAKE &&
                    p.act != OMNI_ACT_LEAKY_RELU))
      return OMNI_ERR_UNSUPPORTED;
    if (a->c_in % (32 * k_splits) || k_splits > 64) return OMNI_ERR_UNSUPPORTED;
    if (kernel != OMNI_CONV_KERNEL_AUTO && kernel != OMNI_CONV_KERNEL_DMA)
      return OMNI_ERR_UNSUPPORTED;
    const int64_t slice = positions * a->n_cols;
    if (slice * 4 > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
    if (launch && (!workspace || !aligned16(workspace) || workspace_bytes < k_splits * slice * 4))
      return OMNI_ERR_INVALID_ARG;
    p.k_splits = (int)k_splits;
    p.partial = workspace;
  }
  Choice ch;
  ch.force = config;
  ch.launch = launch;
  // only the LDS-DMA tiles write split-K partials: a split call no DMA tile fits is refused
  // here, never handed to a family that would write the whole conv into out and leave the
  // reduction summing partials nobody wrote
  int family = k_splits > 1 ? OMNI_CONV_KERNEL_DMA : kernel;
  int r = dispatch(p, x_f32, fp8, fuse2, family, ch, reinterpret_cast<hipStream_t>(stream));
  if (r == OMNI_OK && launch && k_splits > 1) {
    const int quads = (int)(positions * a->n_cols / 4);
    hipLaunchKernelGGL(p.k_splits == 4 ? splitk_reduce_kernel<4> : splitk_reduce_kernel<0>,
                       dim3((unsigned)((quads + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), p.partial, p.k_splits,
                       positions * a->n_cols, p.n_cols, p.c_out, p.length, quads, p.wscale,
                       p.bias, p.act, p.act_a, p.act_b, p.slope, p.out, p.out_bf16, p.o_sb,
                       p.o_st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) r = OMNI_ERR_LAUNCH;
  }
  if (r == OMNI_OK) {
    if (kernel_out) *kernel_out = family;
    if (config_out) *config_out = ch.chosen;
    if (count_out) *count_out = ch.count;
    if (workgroups_out) *workgroups_out = ch.workgroups;
  }
  return r;
}

}  // namespace

extern "C" int omni_conv1d_fused(const omni_conv_args* a, omni_stream_t stream) {
  return conv_entry(a, OMNI_CONV_KERNEL_AUTO, 0, true, nullptr, nullptr, nullptr, nullptr, stream);
}

extern "C" int omni_conv1d_fused_with(const omni_conv_args* a, int kernel, int config,
                                      omni_stream_t stream) {
  if (kernel == OMNI_CONV_KERNEL_AUTO || config < 1) return OMNI_ERR_INVALID_ARG;
  return conv_entry(a, kernel, config, true, nullptr, nullptr, nullptr, nullptr, stream);
}

extern "C" int omni_conv1d_splitk(const omni_conv_args* a, int64_t k_splits, float* workspace,
                                  int64_t workspace_bytes, int kernel, int config,
                                  omni_stream_t stream) {
  if ((kernel == OMNI_CONV_KERNEL_AUTO) != (config == 0)) return OMNI_ERR_INVALID_ARG;
  return conv_entry(a, kernel, config, true, nullptr, nullptr, nullptr, nullptr, stream, k_splits,
                    workspace, workspace_bytes);
}

namespace {

constexpr int kScratchDevices = 64;
std::once_flag scratch_once[kScratchDevices];
float* scratch_device_ptr[kScratchDevices];
int scratch_lookup_status[kScratchDevices];

// This GPU's scratch array (the current device): its device address is looked up once per
// device, with that device current, and kept.
int scratch_address(float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return OMNI_ERR_DEVICE;
  }
  if (dev < 0 || dev >= kScratchDevices) return OMNI_ERR_UNSUPPORTED;
  std::call_once(scratch_once[dev], [dev] {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      scratch_lookup_status[dev] = OMNI_ERR_DEVICE;
      return;
    }
    scratch_device_ptr[dev] = static_cast<float*>(ptr);
    scratch_lookup_status[dev] = OMNI_OK;
  });
  *out = scratch_device_ptr[dev];
  return scratch_lookup_status[dev];
}

}  // namespace

extern "C" int omni_conv1d_splitk_noalloc(const omni_conv_args* a, int64_t k_splits, int kernel,
                                          int config, omni_stream_t stream) {
  if (!a || k_splits < 1 || (kernel == OMNI_CONV_KERNEL_AUTO) != (config == 0))
    return OMNI_ERR_INVALID_ARG;
  if (k_splits > 64) return OMNI_ERR_UNSUPPORTED;
  if (a->batch < 0 || a->length < 0 || a->n_cols < 1) return OMNI_ERR_INVALID_ARG;
  // the partials must fit the array (each slice is written whole before the reduction reads it,
  // so nothing in it has to start at zero)
  if (k_splits > 1 && a->batch > 0 && a->length > 0 &&
      (a->batch > kScratchBytes || a->length > kScratchBytes / a->batch ||
       a->n_cols * k_splits > kScratchBytes / 4 / (a->batch * a->length)))
    return OMNI_ERR_UNSUPPORTED;
  float* ws = nullptr;
  const int st = scratch_address(&ws);
  if (st != OMNI_OK) return st;
  return conv_entry(a, kernel, config, true, nullptr, nullptr, nullptr, nullptr, stream, k_splits,
                    ws, kScratchBytes);
}

extern "C" int omni_conv1d_plan(const omni_conv_args* a, int kernel, int config, int* kernel_out,
                                int* config_out, int* configs_in_list, int64_t* workgroups) {
  if (!kernel_out || !config_out) return OMNI_ERR_INVALID_ARG;
  *kernel_out = OMNI_CONV_KERNEL_AUTO;
  *config_out = 0;
  if (configs_in_list) *configs_in_list = 0;
  if (workgroups) *workgroups = 0;
  return conv_entry(a, kernel, config, false, kernel_out, config_out, configs_in_list, workgroups,
                    nullptr);
}
