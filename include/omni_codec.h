/*
 * omni_codec.h — C ABI of the MI355X (gfx950) codec/vocoder decode kernels.
 *
 * Every entry point takes device pointers, explicit int64 sizes and element strides, scalar
 * parameters and a hipStream_t; it enqueues work on that stream, never synchronises with the
 * host, never allocates device memory, and returns an int status (OMNI_OK = 0, otherwise one of
 * the OMNI_ERR_* codes below; omni_codec_error_string names it). Arguments are validated before
 * any launch, so an error leaves every buffer untouched. All entry points are capturable into a
 * hipGraph.
 *
 * Activations are channels-last: element (b, t, c) of a [B, T, C] tensor sits at
 * b * stride_b + t * stride_t + c (channel stride 1) unless an entry point says otherwise.
 *
 * Reference interfaces replaced (paths relative to the SGLang-Omni checkout):
 *   omni_rvq_gather_sum          F.embedding + per-codebook sum: DAC ResidualVectorQuantize
 *                                .from_codes via sglang_omni/models/fishaudio_s2_pro/fish_speech/
 *                                models/dac/rvq.py:374-388; sglang_omni/models/personaplex/
 *                                components/mimi.py:275-280; sglang_omni/models/higgs_tts/
 *                                audio_codec.py:60-78; mean form sglang_omni/models/qwen3_omni/
 *                                components/code2wav.py:443; ordered gather-sum
 *                                sglang_omni/models/moss_tts/channel_embedding.py:13-50
 *   omni_conv1d_fused            channels_last_conv1d / channels_last_conv_transpose1d
 *                                (sglang_omni/utils/channels_last_conv.py:45-120) with the
 *                                epilogue of fused_bias_snake_beta
 *                                (sglang_omni/kernels/bias_snake_beta.py:102-151) and the slot
 *                                history of history_exchange (sglang_omni/kernels/
 *                                codec_state.py:150-181) folded in
 *   omni_residual_stack          the ResidualUnit modules of a DAC DecoderBlock (sglang_omni/
 *                                models/fishaudio_s2_pro/fish_speech/models/dac/
 *                                modded_dac.py:619-643,742-790) as channels_last_decoder.py:
 *                                114-122 runs them
 *   omni_single_output_conv      clamped_single_output_conv (sglang_omni/kernels/
 *                                single_output_conv.py:62-102); tanh form modded_dac.py:829
 *   omni_history_exchange        history_exchange (sglang_omni/kernels/codec_state.py:150-181)
 *   omni_overlap_exchange        overlap_exchange (sglang_omni/kernels/codec_state.py:184-210)
 *   omni_bias_snake_beta         fused_bias_snake_beta (sglang_omni/kernels/bias_snake_beta.py:
 *                                102-151)
 *   omni_snake                   snake_channels_last_kernel (sglang_omni/models/fishaudio_drama3/
 *                                channels_last_decoder.py:35-67,157-184)
 *   omni_snake_beta              fused_snake_beta's launch (sglang_omni/utils/snake_beta.py:
 *                                164-234) with its bitwise eager-chain contract
 *   omni_conv1d_general          channels_last_conv1d / channels_last_conv_transpose1d
 *                                (sglang_omni/utils/channels_last_conv.py:45-120) for grouped,
 *                                strided, padded or odd-channel convs and float32 / fp16
 *   omni_advance_slots           pool.frame_positions.index_put_ at the end of decode_slots
 *                                (sglang_omni/models/qwen3_omni/components/code2wav.py:459)
 *   omni_codec_capabilities      no kernel counterpart; the platform query of
 *                                sglang_omni/platforms/rocm.py:22-131
 *   omni_short_time_spectrum     short_time_spectrum (sglang_omni/models/fun_cosyvoice3/
 *                                hift_kernels.py:116-146,304-330); with centring, the reflect
 *                                padding of HiftChannelsLast.spectrum (hift_channels_last.py:
 *                                108-115) folded in
 *   omni_overlap_add_inverse     overlap_add_inverse (hift_kernels.py:148-191,333-360)
 *   omni_istft_tail              HiftChannelsLast's exp / sin of the last conv's output, inverse
 *                                and clamp (hift_channels_last.py:117-125,269-276) in one launch
 */
#ifndef OMNI_CODEC_H_
#define OMNI_CODEC_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* omni_stream_t;

enum {
  OMNI_OK = 0,
  OMNI_ERR_INVALID_ARG = 1, /* a shape, stride, pointer or flag outside the documented contract */
  OMNI_ERR_UNSUPPORTED = 2, /* a valid request the library has no kernel for */
  OMNI_ERR_LAUNCH = 3,      /* the HIP runtime refused the launch */
  OMNI_ERR_DEVICE = 4       /* a HIP device query failed */
};

enum {
  OMNI_DTYPE_F32 = 0,
  OMNI_DTYPE_BF16 = 1,
  OMNI_DTYPE_F16 = 2,
  OMNI_DTYPE_FP8_E4M3 = 3, /* OCP e4m3fn, the torch.float8_e4m3fn encoding */
  OMNI_DTYPE_I32 = 4,
  OMNI_DTYPE_I64 = 5
};

enum {
  OMNI_ACTIVATION_NONE = 0,
  OMNI_ACTIVATION_SNAKE = 1, /* v + b[c] * sin(a[c] * v)^2: Snake1d (a = alpha, b = 1/(alpha+1e-9))
                                or SnakeBeta (a = exp(alpha), b = 1/(exp(beta)+1e-9)) */
  OMNI_ACTIVATION_LEAKY_RELU = 2,
  OMNI_ACTIVATION_TANH = 3,
  OMNI_ACTIVATION_CLAMP = 4 /* clamp(v, -1, 1), NaN propagated */
};

/* omni_rvq_gather_sum flags */
enum {
  OMNI_RVQ_MEAN = 1,  /* divide the float32 sum by the number of codebooks once at the end */
  OMNI_RVQ_CLAMP = 2  /* codes above V-1 read entry V-1 (rvq.py:374-388); without it, and for
                         negative codes always, an out-of-range code adds nothing */
};

const char* omni_codec_error_string(int status);
int omni_codec_abi_version(void); /* 11: float16 mix streams (omni_conv_args.mix_a / mix_b in
                                       residual_dtype); 10: omni_gemm */

/* Device facts the host layer sizes its launches with: the gfx arch name (e.g. "gfx950"), LDS
   bytes per workgroup and compute-unit count. */
int omni_codec_capabilities(int device, char* arch, int arch_capacity, int64_t* lds_bytes,
                            int64_t* compute_units);

/*
 * RVQ dequantize: out[b, t, :] = sum_{k=0}^{K-1} E_k[codes[b, k, t]], accumulated in float32 in
 * the order k = 0 .. K-1 (bit-identical to the sequential float32 sum), rounded once to
 * out_dtype. codes int32/int64 with strides (b, k, t); codebooks [K, V, D] contiguous, float32 or
 * bf16; out float32 or bf16 at b * out_stride_b + t * out_stride_t + d * out_stride_d.
 */
int omni_rvq_gather_sum(const void* codes, int codes_dtype, int64_t batch, int64_t num_codebooks,
                        int64_t frames, int64_t codes_stride_b, int64_t codes_stride_k,
                        int64_t codes_stride_t, const void* codebooks, int table_dtype,
                        int64_t codebook_size, int64_t dim, void* out, int out_dtype,
                        int64_t out_stride_b, int64_t out_stride_t, int64_t out_stride_d,
                        int flags, omni_stream_t stream);

/*
 * One fused convolution over channels-last activations, on bf16 MFMA:
 *
 *   u[b, p, ci] = in_act(x[b, p, ci])   rounded to bf16 (x bf16 or float32; in_act is applied
 *                                       to x only, never to history or padding, which are zero
 *                                       or already activated)
 *   acc[b, i, n] = sum_{j < taps} sum_{ci < c_in} W[n, j, ci] * u[b, i + j * dilation - left_pad, ci]
 *   v = acc * weight_scale[n] (fp8 weights only) + bias[n % c_out]
 *   with weight2 (a second, k = 1 conv fused behind the first; needs n_cols == c_out, and the
 *   second conv maps c_out -> c_out channels):
 *     h[b, i, n] = mid_act(v) rounded to bf16
 *     v = (sum_{n'} W2[n, n'] * h[b, i, n']) * weight2_scale[n] (fp8 only) + bias2[n]
 *   v = v (+ residual[b, i, n])
 *   v = ((mix_a[b, i, n] + mix_b[b, i, n]) + v) * mix_scale      (optional, mix_a != NULL)
 *   sum_out[b, i, n] = v            (optional; float32, or float16 rounded to nearest even)
 *   out[b, i, n] = act(v)           (bf16 or float32; optional when sum_out is given)
 *
 * for i < length and n < n_cols. x holds x_length positions per row (x_length = 0 means length);
 * the residual, mix and sum_out tensors share the residual strides; residual, mix and sum_out
 * are float32, or float16 with residual_dtype = OMNI_DTYPE_F16 (residual streams kept in half
 * precision between launches, widened exactly and added in float32); sum_out may alias residual
 * (each element is read before it is written by the same thread) but no output may alias x. A
 * causal Conv1d is taps = k, left_pad = (k-1)*d; a ConvTranspose1d of stride s is its polyphase
 * form (n = phase * c_out + co, so out viewed as [B, length * s, c_out] is the transposed conv's
 * output), see the packing helpers of the host layer. Inputs left of position 0 come from the
 * slot history (below) or are zero; inputs at or past x_length are zero. The batch rows are one
 * position space for tiling, so short rows (streaming chunks) share weight tiles.
 *
 * weight: packed [ceil(c_in/32)][n_cols][taps][32] (ci = 32 * chunk + lane, zero past c_in),
 * bf16, or fp8-e4m3 with weight_scale[n_cols] float32; weight2 the same layout with taps = 1 and
 * c_in = n_cols = c_out, in the same dtype (weight2_scale for fp8).
 *
 * Streaming history (hist_pool != NULL; requires left_pad == (taps-1)*dilation): the pool is
 * bf16 [slots][2][left_pad][c_in] of activated inputs u; row b reads the copy
 * (slot_parity[s] & 1) of slot s = slot_index[b] (zeros instead when history_cold) as positions
 * -left_pad .. -1, and writes the last left_pad samples of (history ++ u) to the other copy.
 * omni_advance_slots flips the parity once every conv of a decode step has run.
 */
typedef struct omni_conv_args {
  const void* x;
  int x_dtype; /* OMNI_DTYPE_BF16 or OMNI_DTYPE_F32 */
  int64_t x_stride_b, x_stride_t;
  int64_t batch, length, c_in;
  int64_t x_length;
  int in_activation; /* OMNI_ACTIVATION_NONE, _SNAKE or _LEAKY_RELU, per input channel */
  const float* in_act_a;
  const float* in_act_b;
  float in_act_slope;
  const void* weight;
  int weight_dtype;
  const float* weight_scale;
  int64_t n_cols, c_out, taps, dilation, left_pad;
  const float* bias;
  const void* weight2; /* optional fused k = 1 conv */
  const float* weight2_scale;
  const float* bias2;
  int mid_activation;
  const float* mid_act_a;
  const float* mid_act_b;
  float mid_act_slope;
  const void* hist_pool;
  const int64_t* slot_index;
  const int64_t* slot_parity;
  int64_t hist_num_slots;   /* slots in the pool; a row whose slot is outside [0, slots) reads
                               zeros and writes no history */
  int64_t hist_slot_stride; /* elements between consecutive slots (= 2 * left_pad * c_in) */
  int history_cold;
  const void* residual; /* float32, or float16 (residual_dtype) */
  int64_t residual_stride_b, residual_stride_t;
  const void* mix_a; /* float32, or float16 (residual_dtype) */
  const void* mix_b;
  float mix_scale;
  void* sum_out; /* float32, or float16 (residual_dtype) */
  void* out;
  int out_dtype;
  int64_t out_stride_b, out_stride_t;
  int activation;
  const float* act_a;
  const float* act_b;
  float act_slope;
  /* ABI version 9: OMNI_DTYPE_F32 (0) or OMNI_DTYPE_F16, the dtype of residual and sum_out */
  int residual_dtype;
} omni_conv_args;

int omni_conv1d_fused(const omni_conv_args* args, omni_stream_t stream);

/*
 * Kernel families of omni_conv1d_fused, each with a list of tile configurations (output columns x
 * positions per workgroup, waves, staged rows) that the call picks from by problem size:
 *   OMNI_CONV_KERNEL_DMA         LDS-DMA staged; bf16 operand used as is (no in_activation), c_in
 *                                a multiple of 32, no weight2; taps 1, 2 or 7 with bf16 or E4M3
 *                                weights: a list of 4 per tap count (bf16 k = 7 at 128 columns:
 *                                1, at 64 or fewer: 3); taps 3 and 11 with bf16 weights at 64
 *                                columns or fewer (4 and 3), at a multiple of 128 or of 96
 *                                columns (taps 3: 2 each) or at 128 (taps 11: 2)
 *   OMNI_CONV_KERNEL_STAGED      register-staged, taps <= 7, any operand mode and weight dtype;
 *                                10 configurations
 *   OMNI_CONV_KERNEL_STAGED11    register-staged, taps <= 11, bf16 weights, x bf16; 10
 *   OMNI_CONV_KERNEL_FUSED_UNIT  the weight2 form (96 or 192 columns): full and short-row tiles
 * omni_conv1d_fused_with runs the same arithmetic with the family and the list's config-th entry
 * (1-based) named by the caller (OMNI_ERR_UNSUPPORTED when they cannot serve the call); the
 * results of every configuration agree to float32 summation order. omni_conv1d_plan reports,
 * without launching and without touching any pointer, the family, the entry, the list's length and
 * the workgroup count that omni_conv1d_fused (kernel = OMNI_CONV_KERNEL_AUTO, config = 0) or
 * omni_conv1d_fused_with (kernel, config) would launch; *kernel_out = OMNI_CONV_KERNEL_AUTO when
 * the call is empty. No reference counterpart: these exist so tests can hold every configuration
 * against the float64 conv, and so a caller can see which one its shapes take.
 */
enum {
  OMNI_CONV_KERNEL_AUTO = 0,
  OMNI_CONV_KERNEL_DMA = 1,
  OMNI_CONV_KERNEL_STAGED = 2,
  OMNI_CONV_KERNEL_STAGED11 = 3,
  OMNI_CONV_KERNEL_FUSED_UNIT = 4
};

int omni_conv1d_fused_with(const omni_conv_args* args, int kernel, int config,
                           omni_stream_t stream);

/*
 * Split-K form of a k = 1 conv used as a GEMM (replaces the plain GEMMs of the code2wav
 * pre-transformer, `F.linear` in sglang_omni/models/qwen3_omni/components/code2wav.py:266,311,
 * 318,322, and of the ConvNeXt blocks' pointwise convs, incremental_codec.py:174-175), or of a
 * k = 7 conv with few output positions (a decoder's input conv over a streaming step, the
 * `CausalConvNet` of modded_dac.py:566-572): the LDS-DMA kernel runs k_splits slices of the
 * 32-channel chunks of each tile (the k = 7 form staging its history rows per slice and writing
 * the new history of its own chunks), each writing its float32 partial tile [positions][n_cols]
 * into `workspace` (k_splits * batch * length * n_cols floats, 16-byte aligned), then a
 * reduction sums the slices in slice order and applies the bias, the output activation and the
 * bf16 / float32 store. The summation order depends on (c_in, taps, k_splits) only, never on the
 * row count, so a caller that fixes k_splits per layer gets the same bits for a row whatever
 * batch it runs in. Takes: taps = 1 or 7, a bf16 operand without in_activation, bf16 weights,
 * history (k = 7), activation NONE, SNAKE or LEAKY_RELU; no weight2, residual, mix or sum_out;
 * c_in a multiple of 32 * k_splits. k_splits = 1 is omni_conv1d_fused. kernel / config as in
 * omni_conv1d_fused_with (OMNI_CONV_KERNEL_AUTO / 0, or OMNI_CONV_KERNEL_DMA and an entry of its
 * list). k_splits > 1 runs on the LDS-DMA family only: a call that none of its split tiles can
 * hold (e.g. k = 7 over many rows of a few positions each, whose history rows overflow the
 * tile's staged rows) returns OMNI_ERR_UNSUPPORTED before any launch and leaves out untouched;
 * the caller then runs the conv unsplit (omni_conv1d_fused).
 */
int omni_conv1d_splitk(const omni_conv_args* args, int64_t k_splits, float* workspace,
                       int64_t workspace_bytes, int kernel, int config, omni_stream_t stream);

/*
 * omni_conv1d_splitk without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference. The float32 partials go to a static device array of 64 MiB
 * per GPU (OMNI_SPLITK_SCRATCH_BYTES; the current device's, whose address is looked up once per
 * device), held until the process ends; the call allocates and frees nothing. Partials beyond
 * the array (k_splits * batch * length * n_cols * 4 bytes) return OMNI_ERR_UNSUPPORTED before
 * any launch. Every call on one GPU shares its array: calls that overlap on one GPU (other
 * streams, other threads) race; the stream must belong to the current device. Same arithmetic,
 * hence the same bits, as omni_conv1d_splitk.
 */
#define OMNI_SPLITK_SCRATCH_BYTES (64ll << 20)
int omni_conv1d_splitk_noalloc(const omni_conv_args* args, int64_t k_splits, int kernel, int config,
                               omni_stream_t stream);
/*
 * omni_resblock_pair: a ResBlock pair of a 32-channel HiFiGAN stage in one launch, h = act1(c1(x))
 * kept in LDS and y = c2(h) through c2's epilogue (hift_layers.py:95-110: xt = c1(act(x)), xt =
 * c2(act(xt)), x = xt + x). c1 describes the first conv (x, weights, bias, dilation d <= 5,
 * activation NONE or LEAKY_RELU, no output, residual or mix); c2 the second (no x: its operand is
 * h; bias, residual, mix, sum_out, out and activation as omni_conv1d_fused takes them). Both 32
 * channels, bf16 weights and operand, k = 3, 7 or 11 with "same" padding (left_pad = (k-1)*d/2 and
 * (k-1)/2), no history, input activation or fused second conv; else OMNI_ERR_UNSUPPORTED. The
 * result equals omni_conv1d_fused of c1 (into a bf16 h) then of c2, bit for bit.
 */
int omni_resblock_pair(const omni_conv_args* c1, const omni_conv_args* c2, omni_stream_t stream);
int omni_conv1d_plan(const omni_conv_args* args, int kernel, int config, int* kernel_out,
                     int* config_out, int* configs_in_list, int64_t* workgroups);

/*
 * The residual units of a DAC decoder block in one launch (Snake -> conv k = 7, dilation d ->
 * Snake -> conv k = 1 -> + x, for each unit in turn), the residual stream kept in float32 (x read
 * as float32 or float16, x_out written as either, x_dtype):
 *
 *   x_0 = x
 *   for each unit k:
 *     u_k = in_act_k(x_k) rounded to bf16               (Snake with unit.in_act_a / in_act_b)
 *     v   = sum_{j < 7} sum_ci W1_k[n, j, ci] * u_k[b, i + (j - 6) * d_k, ci] * w1_scale + bias1
 *     h   = Snake(mid_act_a, mid_act_b)(v) rounded to bf16
 *     x_{k+1} = (sum_n' W2_k[n, n'] * h[n']) * w2_scale + bias2 + x_k
 *   out   = Snake(out_act_a, out_act_b)(x_last) rounded to bf16   (the next layer's operand)
 *   x_out = x_last                                        (optional; float32 or float16)
 *   final_out = the decoder's final conv of out (optional, below)
 *
 * with the arithmetic of one omni_conv1d_fused residual-unit call per unit, so with a float32
 * residual stream the results are the same bits (with a float16 one the calls round x between
 * units, which the stack does not). Weights use omni_conv1d_fused's packing ([C/32][C][7][32] and [C/32][C][32],
 * bf16, or fp8-e4m3 with per-column scales). Each unit's dilated conv keeps its own streaming
 * history (unit.hist_pool, bf16 [slots][2][6 * d_k][C], the omni_conv1d_fused contract with
 * the shared slot_index / slot_parity / history_cold). channels = 96; x, out and x_out are
 * [B, L, C] with channel stride 1 and must not alias.
 *
 * Replaces the three ResidualUnit modules of a DecoderBlock
 * (sglang_omni/models/fishaudio_s2_pro/fish_speech/models/dac/modded_dac.py:619-643,742-790) as
 * the channels-last decoder runs them (sglang_omni/models/fishaudio_drama3/
 * channels_last_decoder.py:114-122).
 */
typedef struct omni_residual_unit {
  const void* weight1;
  const float* weight1_scale;
  const float* bias1;
  int64_t dilation;
  const float* in_act_a;
  const float* in_act_b;
  const float* mid_act_a;
  const float* mid_act_b;
  const void* weight2;
  const float* weight2_scale;
  const float* bias2;
  void* hist_pool;
  int64_t hist_slot_stride;
} omni_residual_unit;

#define OMNI_MAX_RESIDUAL_UNITS 4

typedef struct omni_residual_stack_args {
  const void* x; /* float32, or float16 (x_dtype) */
  int64_t x_stride_b, x_stride_t;
  int64_t batch, length, channels;
  int weight_dtype;
  int num_units;
  omni_residual_unit units[OMNI_MAX_RESIDUAL_UNITS];
  const int64_t* slot_index;
  const int64_t* slot_parity;
  int64_t hist_num_slots;
  int history_cold;
  const float* out_act_a;
  const float* out_act_b;
  void* out; /* bf16 */
  int64_t out_stride_b, out_stride_t;
  void* x_out; /* optional; float32, or float16 (x_dtype) */
  int64_t x_out_stride_b, x_out_stride_t;
  /* Optional (final_weight != NULL): the decoder's conv to one channel fused behind the stack,
   * over u = Snake(out_act)(x_last) rounded to bf16:
   *   final_out[b, i] = final_act(final_bias + sum_{j < taps} sum_c
   *                               final_weight[j * C + c] * u[b, i + j - (taps - 1), c])
   * on the matrix cores: the weights are rounded to bf16 (the decoder's are bf16 values) and the
   * products summed in float32 in the MFMA's order, one fixed order per position (so any split
   * of positions or rows gives the same bits; they can differ from omni_single_output_conv's in
   * the last places). taps = final_taps <= 8; positions left of 0 come from final_hist_pool (bf16
   * [slots][2][taps - 1][C], the omni_conv1d_fused history contract, sharing slot_index,
   * slot_parity and history_cold) or are zero. out may be NULL when final_weight is given. */
  const float* final_weight;
  const float* final_bias;
  int64_t final_taps;
  int final_activation; /* OMNI_ACTIVATION_TANH, _CLAMP or _NONE */
  void* final_hist_pool;
  int64_t final_hist_slot_stride;
  float* final_out; /* float32, element (b, i) at b * final_out_stride_b + i */
  int64_t final_out_stride_b;
  /* ABI version 5: the per-channel coefficient rows the launch would otherwise compute in every
     workgroup, precomputed by omni_residual_stack_coefficients for these units (16-byte
     aligned), or NULL */
  const float* coef_table;
  /* ABI version 9: OMNI_DTYPE_F32 (0) or OMNI_DTYPE_F16, the dtype of x and x_out (the stack
     keeps x in float32 between its units and rounds x_out once) */
  int x_dtype;
} omni_residual_stack_args;

/* Fills table[(num_units * 8 + 2) * channels] (float32, device, 16-byte aligned) with the
   coefficient rows of a's units and output Snake (a's weights, activations and scales; its
   activations / histories / outputs are not read). Call once per set of weights; pass the table
   as coef_table to every omni_residual_stack call with those weights. */
int omni_residual_stack_coefficients(const omni_residual_stack_args* a, float* table,
                                     int64_t table_floats, omni_stream_t stream);

int omni_residual_stack(const omni_residual_stack_args* args, omni_stream_t stream);

/*
 * Conv from channels-last activations to one output channel, stride 1, undilated:
 *   u = in_act(x) (OMNI_ACTIVATION_NONE or _SNAKE with per-channel in_act_a / in_act_b)
 *   out[b, i] = act(bias + sum_{j < taps} sum_c weight[j * channels + c] * u[b, i + j - left_pad, c])
 * accumulated in float32 in one fixed order per position (so any split of positions or rows gives
 * identical bits) and rounded once. x points at position 0 and holds `length` positions (later
 * ones read as zero); when context_in_buffer is set, the left_pad positions before it are valid
 * memory (the reference's padded input); otherwise they come from the slot history (bf16 pool
 * [slots][2][taps-1][channels] of activated inputs, same parity rule as omni_conv1d_fused; needs
 * left_pad = taps-1) or are zero. With an input activation or a history the activated inputs are
 * rounded to bf16 (the decoder's operands and its history); otherwise they are used exactly.
 * activation is OMNI_ACTIVATION_TANH or _CLAMP or _NONE. x dtype bf16, f16 or f32, channels a
 * multiple of 4 (of 8 with an activation or history); out [B, 1, length] at b * out_stride_b + i,
 * dtype of out_dtype.
 */
int omni_single_output_conv(const void* x, int x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                            int64_t batch, int64_t length, int64_t channels, int context_in_buffer,
                            int in_activation, const float* in_act_a, const float* in_act_b,
                            const float* weight, const float* bias, int64_t taps, int64_t left_pad,
                            const void* hist_pool, const int64_t* slot_index,
                            const int64_t* slot_parity, int64_t hist_num_slots,
                            int64_t hist_slot_stride, int history_cold, int activation,
                            void* out, int out_dtype,
                            int64_t out_stride_b, omni_stream_t stream);

/*
 * history_exchange, in place, any element strides: padded[r, :H] = pool[slot_index[r]] (zeros
 * when cold), padded[r, H + new_samples:] = 0, then pool[slot_index[r]] = padded[r, new_samples :
 * new_samples + H] (the values before this call's writes). dtype bf16, f16 or f32; bitwise.
 * Rows whose slot is outside [0, num_slots) are left untouched.
 */
int omni_history_exchange(void* padded, int dtype, int64_t rows, int64_t padded_samples,
                          int64_t channels, int64_t padded_stride_row,
                          int64_t padded_stride_sample, int64_t padded_stride_channel,
                          void* history_pool, int64_t num_slots, int64_t history_samples,
                          int64_t pool_stride_slot,
                          int64_t pool_stride_sample, int64_t pool_stride_channel,
                          const int64_t* slot_index, int64_t new_samples, int is_cold,
                          omni_stream_t stream);

/*
 * overlap_exchange, in place: output[r, :O] += pool[slot_index[r]] (in float32, rounded once; not
 * when cold), then pool[slot_index[r]] = output[r, emitted : emitted + O] (values before the add).
 * Requires emitted_samples >= O. dtype bf16, f16 or f32; bitwise. Rows whose slot is outside
 * [0, num_slots) are left untouched.
 */
int omni_overlap_exchange(void* output, int dtype, int64_t rows, int64_t channels,
                          int64_t output_stride_row, int64_t output_stride_sample,
                          int64_t output_stride_channel, void* overlap_pool, int64_t num_slots,
                          int64_t overlap_samples, int64_t pool_stride_slot,
                          int64_t pool_stride_sample, int64_t pool_stride_channel,
                          const int64_t* slot_index, int64_t emitted_samples, int is_cold,
                          omni_stream_t stream);

/*
 * fused_bias_snake_beta: t = round(conv + bias); if residual: t = round(t + residual);
 * sum_out = t; out = round(t + round(inverse_beta * round(round(sin(round(t * alpha_scale)))^2)))
 * with every round to `dtype` (bf16 or f16), as the eager op chain rounds. conv and out rows
 * (stride_b apart) are [length, channels] contiguous; residual and sum_out are contiguous
 * [batch, length, channels]; bias / alpha_scale / inverse_beta are [channels] of param_dtype.
 */
int omni_bias_snake_beta(const void* conv, int64_t conv_stride_b, int64_t batch, int64_t length,
                         int64_t channels, const void* bias, const void* alpha_scale,
                         const void* inverse_beta, int param_dtype, const void* residual,
                         void* sum_out, void* out, int64_t out_stride_b, int dtype,
                         omni_stream_t stream);

/*
 * Standalone Snake family on [B, T, C] (channels_last != 0) or [B, C, T] rows, dtype bf16, f16 or
 * f32: y = x + b[c] * sin(a[c] * x)^2. round_intermediates = 0 computes in float32 and rounds once
 * (Snake1d's channels-last kernel); 1 rounds after every op like the eager SnakeBeta chain.
 * x and y have identical contiguous layouts.
 */
int omni_snake(const void* x, void* y, int dtype, int64_t batch, int64_t frames,
               int64_t channels, int channels_last, const float* a, const float* b,
               int round_intermediates, omni_stream_t stream);

/*
 * fused_snake_beta with the module's parameters (sglang_omni/utils/snake_beta.py:200-234): alpha
 * and beta are SnakeBeta's log-scale [channels] parameters in x's dtype (bf16 or f16), read on the
 * device at every launch, eps its no_div_by_zero; every op of the eager chain rounds to the dtype:
 *   a = exp(alpha), e = exp(beta), t = e + eps, r = 1 / t, y = x + r * sin(x * a)^2.
 * x is [B, C, T] contiguous (channels_last = 0) or the [B, C, T] view of a contiguous [B, T, C]
 * (channels_last = 1); y has x's layout and must not overlap it.
 */
int omni_snake_beta(const void* x, void* y, int dtype, int64_t batch, int64_t channels,
                    int64_t frames, int channels_last, const void* alpha, const void* beta,
                    int param_dtype, float eps, omni_stream_t stream);

/*
 * Conv1d / ConvTranspose1d of channels-last activations in the general form of the reference's
 * channels-last conv API (sglang_omni/utils/channels_last_conv.py:45-120), for what the MFMA
 * kernel does not take: any channel counts, groups, stride, dilation and zero padding, float32,
 * bf16 or f16 activations, weights and bias of that dtype, float32 accumulation (taps ascending,
 * then the group's input channels), one rounding to the dtype:
 *   conv        y[b, i, co] = bias[co] + sum_{j, c} W[co, c, j] x[b, i * stride + j * dilation -
 *               pad_left, g * C_in / groups + c]
 *   transposed  y[b, i, co] = bias[co] + sum_{j, c} W[g * C_in / groups + c, co - g * C_out /
 *               groups, j] x[b, q, g * C_in / groups + c] over q * stride + j * dilation = i +
 *               pad_left
 * with g = co / (C_out / groups) and inputs outside [0, length_in) zero. x, W and y at the given
 * element strides (W in the module's layout: [C_out, C_in / groups, k] for a conv, [C_in,
 * C_out / groups, k] for a transposed conv); y must not overlap x.
 */
int omni_conv1d_general(const void* x, int dtype, int64_t batch, int64_t length_in, int64_t c_in,
                        int64_t x_stride_b, int64_t x_stride_t, int64_t x_stride_c,
                        const void* weight, int64_t taps, int64_t weight_stride0,
                        int64_t weight_stride1, int64_t weight_stride2, const void* bias,
                        int64_t c_out, int64_t groups, int64_t stride, int64_t dilation,
                        int64_t pad_left, int transposed, void* y, int64_t length_out,
                        int64_t y_stride_b, int64_t y_stride_t, int64_t y_stride_c,
                        omni_stream_t stream);

/* slot_parity[slot_index[r]] += 1 for r < rows whose slot is in [0, num_slots), ending a decode
   step (graph-capturable). */
int omni_advance_slots(int64_t* slot_parity, int64_t num_slots, const int64_t* slot_index,
                       int64_t rows, omni_stream_t stream);

/*
 * HiFT's short-time Fourier transform and its inverse (n_fft <= 64, hop divides n_fft,
 * bins = n_fft / 2 + 1; every output summed in one fixed order, float32).
 *
 * omni_short_time_spectrum: spectrum [rows][2 * bins][frames] (real parts, then imaginary) with
 *   spectrum[r, c, f] = sum_{k < n_fft} xp[r, f * hop + k] * basis[c * n_fft + k], where xp is the
 *   signal reflect-padded by n_fft / 2 on both sides when center (needs samples > n_fft / 2), else
 *   the signal itself (already padded); frames = (padded_samples - n_fft) / hop + 1. basis is
 *   [2 * bins][n_fft]: the windowed cosines, then the windowed negative sines.
 * omni_overlap_add_inverse: torch.istft (center = True, one-sided) of real / imag
 *   [rows][bins][frames]: out[r, i] = (sum over the frames f covering padded position
 *   p = i + n_fft / 2 of sum_{b < bins} real[r, b, f] * basis[b, t] + imag[r, b, f] *
 *   basis[bins + b, t]) / (sum over the same frames of squared_window[t]), t = p - f * hop, for
 *   i < hop * (frames - 1); basis [2 * bins][n_fft] is the one-sided inverse's windowed cosines and
 *   negative sines (bins 1 .. bins-2 doubled) divided by n_fft.
 * omni_istft_tail: the same inverse of magnitude = min(exp(h[r, f, b]), magnitude_clip) and
 *   phase = sin(h[r, f, bins + b]) (real = magnitude * cos(phase), imag = magnitude * sin(phase)),
 *   h the vocoder's last conv output, channels-last float32 at r * h_stride_row +
 *   f * h_stride_frame + c, then clamped to [-audio_limit, audio_limit].
 */
int omni_short_time_spectrum(const float* signal, int64_t rows, int64_t samples,
                             int64_t signal_stride_row, int center, const float* basis,
                             int64_t bins, int64_t n_fft, int64_t hop, float* spectrum,
                             int64_t frames, omni_stream_t stream);
int omni_overlap_add_inverse(const float* real, const float* imag, int64_t rows, int64_t bins,
                             int64_t frames, const float* basis, const float* squared_window,
                             int64_t n_fft, int64_t hop, float* out, int64_t out_stride_row,
                             omni_stream_t stream);
int omni_istft_tail(const float* h, int64_t rows, int64_t frames, int64_t h_stride_row,
                    int64_t h_stride_frame, const float* basis, const float* squared_window,
                    int64_t bins, int64_t n_fft, int64_t hop, float magnitude_clip,
                    float audio_limit, float* out, int64_t out_stride_row, omni_stream_t stream);

/*
 * Waveform egress (no reference counterpart as one call: it replaces the per-request
 * `slot.view(samples).copy_(waveform)` staging of code2wav_scheduler.py:756-800 and the float32 ->
 * PCM16 encoding of serve/realtime/session_bridge.py:86-88). Packs rows of a float32 waveform
 * (wave[r * wave_stride_row + i], i < samples) into out[r * out_stride_row + i] so that one
 * device-to-host copy moves a whole decode step:
 *   OMNI_EGRESS_F32    out is float32, the samples unchanged;
 *   OMNI_EGRESS_PCM16  out is int16: (int16) trunc(clip(v, -1, 1) * 32767.0f), NaN -> 0.
 * row_samples (nullable, device int64[rows]) stops row r after min(row_samples[r], samples)
 * samples; the rest of that output row is not written.
 */
enum omni_egress_format {
  OMNI_EGRESS_F32 = 0,
  OMNI_EGRESS_PCM16 = 1
};

int omni_waveform_egress(const float* wave, int64_t rows, int64_t samples,
                         int64_t wave_stride_row, const int64_t* row_samples, int format,
                         void* out, int64_t out_stride_row, omni_stream_t stream);

/*
 * The Qwen3-Omni code2wav front (pre-transformer and ConvNeXt upsamplers): the ops around its
 * plain GEMMs. Activations are bf16 rows (GEMM operands / outputs) and float32 residual streams.
 *
 * omni_rms_norm_residual: per row of h [rows][channels] float32 (contiguous): if delta, h +=
 *   scale[c] * delta[row, c] (the layer-scaled residual add, code2wav.py:300-324's addcmul);
 *   then normed[row, c] = weight[c] * h[row, c] / sqrt(mean_c(h^2) + eps) as bf16 (rmsnorm).
 *   channels a multiple of 256, at most 4096.
 * omni_rope_kv_write: qkv [batch * frames][qkv_stride] bf16 holds q (heads * head_dim), k, v
 *   (kv_heads * head_dim each); q and k get the neox rotary embedding in place at position
 *   start(b) + t, angle = position * inv_freq[i] in float32 (start(b) = 0 if cold, else
 *   positions[slot_index[b]]); with key_ring / value_ring ([slots * ring_frames][kv_heads *
 *   head_dim] bf16) the rotated k and the v of each frame also go to ring row
 *   slot * ring_frames + position % ring_frames (apply_rope_inplace_with_kvcache,
 *   code2wav.py:205-215).
 * omni_window_attention: out[b * frames + t, h * 64 + d] (bf16) = softmax over the keys at
 *   positions p with 0 <= P - p < window (P the query's position) of scale * q . k, times v;
 *   keys / values from the rings (which must hold the window before the new frames, ring_frames >=
 *   window - 1 + frames) or, for a first decode (cold, rings NULL), from qkv itself
 *   (code2wav.py:227-246,278-298). head_dim 64, window <= 113 (the window and 16 queries' keys sit in LDS).
 * omni_silu_mul: out[row, i] = silu(gate_up[row, i]) * gate_up[row, inter + i], bf16.
 * omni_dwconv_layernorm: ConvNeXt's depthwise causal conv (7 taps, weight [7][channels]
 *   float32, tap 6 on the current sample) over x [batch][length][channels] float32 with slot
 *   history (pool [slots][2][6][channels] float32, copy slot_parity & 1 read, the other written),
 *   plus bias, then LayerNorm(eps) with ln_weight / ln_bias, written as bf16
 *   (incremental_codec.py:160-175, modeling_qwen3_omni_moe.py:3231-3264). A row's samples
 *   (length * channels * 4 bytes) below 2 GiB, else OMNI_ERR_UNSUPPORTED.
 * omni_bias_gelu: y = GELU(y + bias[col]) in place (erf form), bf16.
 * omni_bias_scale_residual: r[row, c] += gamma[c] * (y[row, c] + bias[c]) (r float32
 *   contiguous, y bf16); if out, also out[row, c] = bf16(r[row, c]).
 * omni_advance_positions: positions[slot_index[r]] = (cold ? 0 : positions[slot_index[r]]) +
 *   new_frames, the end of a slot decode (code2wav.py:459).
 */
int omni_rms_norm_residual(float* h, int64_t rows, int64_t channels, const void* delta,
                           int64_t delta_stride, const float* scale, const float* weight,
                           float eps, void* normed, int64_t normed_stride, omni_stream_t stream);
int omni_rope_kv_write(void* qkv, int64_t batch, int64_t frames, int64_t qkv_stride,
                       int64_t heads, int64_t kv_heads, int64_t head_dim, const float* inv_freq,
                       const int64_t* slot_index, const int64_t* positions, int cold,
                       int64_t num_slots, void* key_ring, void* value_ring, int64_t ring_frames,
                       omni_stream_t stream);
int omni_window_attention(const void* qkv, int64_t batch, int64_t frames, int64_t qkv_stride,
                          int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t window,
                          float scale, const void* key_ring, const void* value_ring,
                          int64_t ring_frames, const int64_t* slot_index,
                          const int64_t* positions, int cold, int64_t num_slots, void* out,
                          int64_t out_stride, omni_stream_t stream);
int omni_silu_mul(const void* gate_up, int64_t rows, int64_t inter, int64_t in_stride, void* out,
                  int64_t out_stride, omni_stream_t stream);
int omni_dwconv_layernorm(const float* x, int64_t batch, int64_t length, int64_t channels,
                          int64_t x_stride_b, const float* weight, const float* bias,
                          const float* ln_weight, const float* ln_bias, float eps,
                          float* hist_pool, int64_t hist_slot_stride, const int64_t* slot_index,
                          const int64_t* slot_parity, int64_t num_slots, int cold, void* out,
                          int64_t out_stride_b, omni_stream_t stream);
int omni_bias_gelu(void* y, int64_t rows, int64_t cols, int64_t stride, const float* bias,
                   omni_stream_t stream);
int omni_bias_scale_residual(float* r, int64_t rows, int64_t channels, const void* y,
                             int64_t y_stride, const float* bias, const float* gamma, void* out,
                             int64_t out_stride, omni_stream_t stream);
int omni_advance_positions(int64_t* positions, int64_t num_slots, const int64_t* slot_index,
                           int64_t rows, int64_t new_frames, int cold, omni_stream_t stream);

/*
 * omni_gemm: out = epilogue(a [rows][k] x w^T) for the code2wav front's linear layers, w [n][k]
 * bf16 contiguous (a linear layer's weight [out_features][in_features]), a bf16 rows a_stride
 * elements apart, float32 accumulation over k in one fixed order whatever rows is (a row's result
 * does not depend on the rows batched with it). bias (float32 [n], optional) is added to the
 * accumulator first. Epilogues:
 *   OMNI_GEMM_STORE            out bf16 [rows][n] = acc + bias
 *     (F.linear(normed, qkv_weight), sglang_omni/models/qwen3_omni/components/code2wav.py:267)
 *   OMNI_GEMM_SILU_MUL         out bf16 [rows][n / 2]: w's rows interleaved in blocks of 16,
 *     block 2q the gate rows 16q .. 16q + 15 and block 2q + 1 the matching up rows; out[row, i] =
 *     silu(gate_i) * up_i (silu_and_mul(F.linear(normed, gate_up_weight)), code2wav.py:321)
 *   OMNI_GEMM_GELU             out bf16 [rows][n] = GELU(acc + bias), erf form
 *     (act(pwconv1(normed)), qwen3_omni/components/incremental_codec.py:174-176)
 *   OMNI_GEMM_SCALED_RESIDUAL  out [rows][n] = residual + scale[c] * (acc + bias), one float32
 *     fma per element, stored as float32 or rounded to bf16 (out_dtype); residual (float32) may
 *     be out itself (addcmul(residual, layer_scale, F.linear(...)), code2wav.py:311-326;
 *     residual + gamma * pwconv2(...), incremental_codec.py:174-180)
 * out_dtype is OMNI_DTYPE_BF16, or OMNI_DTYPE_F32 for the scaled residual.
 * k a multiple of 64, n of 64; a, w, bias, residual and scale 16-byte aligned with 16-byte row
 * strides; out rows 8-byte (bf16) or 16-byte (float32) aligned. config 0 picks the tile; 1 - 6
 * force one (1: 64 x 128 of 4 waves, 2: 64 x 64 of 4, 3: 64 x 128 of 8, 4: 64 x 64 of 8 (not
 * for SILU_MUL), 5: 32 x 64 of 4, 6: 64 x 128 of 8 as 4 x 2; columns a multiple of the tile's,
 * else OMNI_ERR_UNSUPPORTED). Every tile gives the same bits. rows = 0 does nothing.
 */
enum {
  OMNI_GEMM_STORE = 0,
  OMNI_GEMM_SILU_MUL = 1,
  OMNI_GEMM_GELU = 2,
  OMNI_GEMM_SCALED_RESIDUAL = 3
};
typedef struct omni_gemm_args {
  const void* a;
  int64_t a_stride;
  const void* w;
  int64_t rows, k, n;
  const float* bias;
  int epilogue;
  int out_dtype;
  int config;
  const float* scale;
  const float* residual;
  int64_t residual_stride;
  void* out;
  int64_t out_stride;
} omni_gemm_args;
int omni_gemm(const omni_gemm_args* args, omni_stream_t stream);

/*
 * omni_gemm_rope_kv: the qkv GEMM with omni_rope_kv_write in its epilogue, one launch for
 * F.linear(normed, qkv_weight) then apply_rope_inplace_with_kvcache (sglang_omni/models/
 * qwen3_omni/components/code2wav.py:267, :205-215). args as for omni_gemm with epilogue
 * OMNI_GEMM_STORE, out_dtype bf16 and n = (heads + 2 kv_heads) * head_dim: out (the qkv rows,
 * rows = batch * frames) gets what omni_gemm then omni_rope_kv_write on out leave there, bit for
 * bit, and the rings what omni_rope_kv_write writes. head_dim 64 (else OMNI_ERR_UNSUPPORTED);
 * n a multiple of 128; config 0 or 1 (64 x 128 tiles of 4 waves) or 6 (of 8 waves).
 */
int omni_gemm_rope_kv(const omni_gemm_args* args, int64_t frames, int64_t heads,
                      int64_t kv_heads, int64_t head_dim, const float* inv_freq,
                      const int64_t* slot_index, const int64_t* positions, int cold,
                      int64_t num_slots, void* key_ring, void* value_ring, int64_t ring_frames,
                      omni_stream_t stream);

/*
 * omni_channel_embedding_sum: MOSS-TTS's fused multi-channel embedding
 * (moss_tts/channel_embedding.py:13-50). out[r, :] = sum over c = 0 .. channels-1, in that
 * order, of tables[c][ids[r, c], :], the running total rounded to `dtype` (bf16, f16 or f32)
 * after every add; ids outside [0, vocab_sizes[c]) add nothing. ids (int32 or int64) at
 * r * id_stride_row + c * id_stride_channel; tables a device array of the channels' table
 * addresses ([vocab_sizes[c]][hidden] each, `dtype`, contiguous); vocab_sizes a device int64
 * array; out [rows][hidden] contiguous. Any hidden width; 16-byte loads and stores are used
 * where hidden % 8 == 0 and the table / output address is 16-byte aligned.
 */
int omni_channel_embedding_sum(const void* token_ids, int ids_dtype, int64_t rows,
                               int64_t channels, int64_t id_stride_row, int64_t id_stride_channel,
                               const uint64_t* tables, const int64_t* vocab_sizes, int dtype,
                               int64_t hidden, void* out, omni_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OMNI_CODEC_H_ */
