"""ctypes binding of the in-tree ``libomni_codec.so`` (the gfx950 HIP kernels' C ABI).

The library is built by ``sglang-omni_amd/csrc/build.py`` (``__graft_entry__.build()``). There is
no fallback: if the library is missing, fails to load, or a call returns a nonzero status, the
caller gets an exception — the decode path never silently runs anything else.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libomni_codec.so"

OK = 0
DTYPE_F32, DTYPE_BF16, DTYPE_F16, DTYPE_FP8_E4M3, DTYPE_I32, DTYPE_I64 = range(6)
ACT_NONE, ACT_SNAKE, ACT_LEAKY_RELU, ACT_TANH, ACT_CLAMP = range(5)
RVQ_MEAN, RVQ_CLAMP = 1, 2
EGRESS_F32, EGRESS_PCM16 = 0, 1

TORCH_TO_OMNI = {
    torch.float32: DTYPE_F32,
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_F16,
    torch.float8_e4m3fn: DTYPE_FP8_E4M3,
    torch.int32: DTYPE_I32,
    torch.int64: DTYPE_I64,
}


class OmniCodecError(RuntimeError):
    """A nonzero status from the native library (``status``; 0 when the error is raised on the
    host before any call)."""

    def __init__(self, message: str, status: int = 0):
        super().__init__(message)
        self.status = status


INVALID_ARG = 1
UNSUPPORTED = 2
ABI_VERSION = 11

# kernel families of omni_conv1d_fused (omni_conv1d_plan / omni_conv1d_fused_with)
CONV_KERNEL_AUTO, CONV_KERNEL_DMA, CONV_KERNEL_STAGED, CONV_KERNEL_STAGED11, CONV_KERNEL_FUSED_UNIT = range(5)
CONV_KERNEL_NAMES = {CONV_KERNEL_DMA: "dma", CONV_KERNEL_STAGED: "staged",
                     CONV_KERNEL_STAGED11: "staged11", CONV_KERNEL_FUSED_UNIT: "fused_unit"}


class ConvArgs(ctypes.Structure):
    """Mirror of ``omni_conv_args`` in include/omni_codec.h (field order and types match)."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int),
        ("x_stride_b", ctypes.c_int64),
        ("x_stride_t", ctypes.c_int64),
        ("batch", ctypes.c_int64),
        ("length", ctypes.c_int64),
        ("c_in", ctypes.c_int64),
        ("x_length", ctypes.c_int64),
        ("in_activation", ctypes.c_int),
        ("in_act_a", ctypes.c_void_p),
        ("in_act_b", ctypes.c_void_p),
        ("in_act_slope", ctypes.c_float),
        ("weight", ctypes.c_void_p),
        ("weight_dtype", ctypes.c_int),
        ("weight_scale", ctypes.c_void_p),
        ("n_cols", ctypes.c_int64),
        ("c_out", ctypes.c_int64),
        ("taps", ctypes.c_int64),
        ("dilation", ctypes.c_int64),
        ("left_pad", ctypes.c_int64),
        ("bias", ctypes.c_void_p),
        ("weight2", ctypes.c_void_p),
        ("weight2_scale", ctypes.c_void_p),
        ("bias2", ctypes.c_void_p),
        ("mid_activation", ctypes.c_int),
        ("mid_act_a", ctypes.c_void_p),
        ("mid_act_b", ctypes.c_void_p),
        ("mid_act_slope", ctypes.c_float),
        ("hist_pool", ctypes.c_void_p),
        ("slot_index", ctypes.c_void_p),
        ("slot_parity", ctypes.c_void_p),
        ("hist_num_slots", ctypes.c_int64),
        ("hist_slot_stride", ctypes.c_int64),
        ("history_cold", ctypes.c_int),
        ("residual", ctypes.c_void_p),
        ("residual_stride_b", ctypes.c_int64),
        ("residual_stride_t", ctypes.c_int64),
        ("mix_a", ctypes.c_void_p),
        ("mix_b", ctypes.c_void_p),
        ("mix_scale", ctypes.c_float),
        ("sum_out", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int),
        ("out_stride_b", ctypes.c_int64),
        ("out_stride_t", ctypes.c_int64),
        ("activation", ctypes.c_int),
        ("act_a", ctypes.c_void_p),
        ("act_b", ctypes.c_void_p),
        ("act_slope", ctypes.c_float),
        ("residual_dtype", ctypes.c_int),
    ]


class ResidualUnitArgs(ctypes.Structure):
    """Mirror of ``omni_residual_unit`` in include/omni_codec.h."""

    _fields_ = [
        ("weight1", ctypes.c_void_p),
        ("weight1_scale", ctypes.c_void_p),
        ("bias1", ctypes.c_void_p),
        ("dilation", ctypes.c_int64),
        ("in_act_a", ctypes.c_void_p),
        ("in_act_b", ctypes.c_void_p),
        ("mid_act_a", ctypes.c_void_p),
        ("mid_act_b", ctypes.c_void_p),
        ("weight2", ctypes.c_void_p),
        ("weight2_scale", ctypes.c_void_p),
        ("bias2", ctypes.c_void_p),
        ("hist_pool", ctypes.c_void_p),
        ("hist_slot_stride", ctypes.c_int64),
    ]


MAX_RESIDUAL_UNITS = 4


class ResidualStackArgs(ctypes.Structure):
    """Mirror of ``omni_residual_stack_args`` in include/omni_codec.h."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_stride_b", ctypes.c_int64),
        ("x_stride_t", ctypes.c_int64),
        ("batch", ctypes.c_int64),
        ("length", ctypes.c_int64),
        ("channels", ctypes.c_int64),
        ("weight_dtype", ctypes.c_int),
        ("num_units", ctypes.c_int),
        ("units", ResidualUnitArgs * MAX_RESIDUAL_UNITS),
        ("slot_index", ctypes.c_void_p),
        ("slot_parity", ctypes.c_void_p),
        ("hist_num_slots", ctypes.c_int64),
        ("history_cold", ctypes.c_int),
        ("out_act_a", ctypes.c_void_p),
        ("out_act_b", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("out_stride_b", ctypes.c_int64),
        ("out_stride_t", ctypes.c_int64),
        ("x_out", ctypes.c_void_p),
        ("x_out_stride_b", ctypes.c_int64),
        ("x_out_stride_t", ctypes.c_int64),
        ("final_weight", ctypes.c_void_p),
        ("final_bias", ctypes.c_void_p),
        ("final_taps", ctypes.c_int64),
        ("final_activation", ctypes.c_int),
        ("final_hist_pool", ctypes.c_void_p),
        ("final_hist_slot_stride", ctypes.c_int64),
        ("final_out", ctypes.c_void_p),
        ("final_out_stride_b", ctypes.c_int64),
        ("coef_table", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int),
    ]


class GemmArgs(ctypes.Structure):
    """Mirror of ``omni_gemm_args`` in include/omni_codec.h."""

    _fields_ = [
        ("a", ctypes.c_void_p),
        ("a_stride", ctypes.c_int64),
        ("w", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("bias", ctypes.c_void_p),
        ("epilogue", ctypes.c_int),
        ("out_dtype", ctypes.c_int),
        ("config", ctypes.c_int),
        ("scale", ctypes.c_void_p),
        ("residual", ctypes.c_void_p),
        ("residual_stride", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("out_stride", ctypes.c_int64),
    ]


GEMM_STORE, GEMM_SILU_MUL, GEMM_GELU, GEMM_SCALED_RESIDUAL = 0, 1, 2, 3

_I64 = ctypes.c_int64
_INT = ctypes.c_int
_PTR = ctypes.c_void_p

# name -> argtypes (every entry point returns int status unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "omni_codec_error_string": [_INT],
    "omni_codec_abi_version": [],
    "omni_codec_capabilities": [_INT, ctypes.c_char_p, _INT, ctypes.POINTER(_I64),
                                ctypes.POINTER(_I64)],
    "omni_rvq_gather_sum": [_PTR, _INT, _I64, _I64, _I64, _I64, _I64, _I64, _PTR, _INT, _I64, _I64,
                            _PTR, _INT, _I64, _I64, _I64, _INT, _PTR],
    "omni_conv1d_fused": [ctypes.POINTER(ConvArgs), _PTR],
    "omni_conv1d_fused_with": [ctypes.POINTER(ConvArgs), _INT, _INT, _PTR],
    "omni_conv1d_splitk": [ctypes.POINTER(ConvArgs), _I64, _PTR, _I64, _INT, _INT, _PTR],
    "omni_conv1d_splitk_noalloc": [ctypes.POINTER(ConvArgs), _I64, _INT, _INT, _PTR],
    "omni_conv1d_plan": [ctypes.POINTER(ConvArgs), _INT, _INT, ctypes.POINTER(_INT),
                         ctypes.POINTER(_INT), ctypes.POINTER(_INT), ctypes.POINTER(_I64)],
    "omni_residual_stack": [ctypes.POINTER(ResidualStackArgs), _PTR],
    "omni_residual_stack_coefficients": [ctypes.POINTER(ResidualStackArgs), _PTR, _I64, _PTR],
    "omni_single_output_conv": [_PTR, _INT, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _PTR, _PTR,
                                _PTR, _PTR, _I64, _I64, _PTR, _PTR, _PTR, _I64, _I64, _INT, _INT,
                                _PTR, _INT, _I64, _PTR],
    "omni_history_exchange": [_PTR, _INT, _I64, _I64, _I64, _I64, _I64, _I64, _PTR, _I64, _I64,
                              _I64, _I64, _I64, _PTR, _I64, _INT, _PTR],
    "omni_overlap_exchange": [_PTR, _INT, _I64, _I64, _I64, _I64, _I64, _PTR, _I64, _I64, _I64,
                              _I64, _I64, _PTR, _I64, _INT, _PTR],
    "omni_bias_snake_beta": [_PTR, _I64, _I64, _I64, _I64, _PTR, _PTR, _PTR, _INT, _PTR, _PTR,
                             _PTR, _I64, _INT, _PTR],
    "omni_snake": [_PTR, _PTR, _INT, _I64, _I64, _I64, _INT, _PTR, _PTR, _INT, _PTR],
    "omni_snake_beta": [_PTR, _PTR, _INT, _I64, _I64, _I64, _INT, _PTR, _PTR, _INT, ctypes.c_float,
                        _PTR],
    "omni_conv1d_general": [_PTR, _INT, _I64, _I64, _I64, _I64, _I64, _I64, _PTR, _I64, _I64, _I64,
                            _I64, _PTR, _I64, _I64, _I64, _I64, _I64, _INT, _PTR, _I64, _I64, _I64,
                            _I64, _PTR],
    "omni_advance_slots": [_PTR, _I64, _PTR, _I64, _PTR],
    "omni_short_time_spectrum": [_PTR, _I64, _I64, _I64, _INT, _PTR, _I64, _I64, _I64, _PTR, _I64,
                                 _PTR],
    "omni_overlap_add_inverse": [_PTR, _PTR, _I64, _I64, _I64, _PTR, _PTR, _I64, _I64, _PTR, _I64,
                                 _PTR],
    "omni_istft_tail": [_PTR, _I64, _I64, _I64, _I64, _PTR, _PTR, _I64, _I64, _I64,
                        ctypes.c_float, ctypes.c_float, _PTR, _I64, _PTR],
    "omni_waveform_egress": [_PTR, _I64, _I64, _I64, _PTR, _INT, _PTR, _I64, _PTR],
    "omni_rms_norm_residual": [_PTR, _I64, _I64, _PTR, _I64, _PTR, _PTR, ctypes.c_float, _PTR,
                               _I64, _PTR],
    "omni_rope_kv_write": [_PTR, _I64, _I64, _I64, _I64, _I64, _I64, _PTR, _PTR, _PTR, _INT, _I64,
                           _PTR, _PTR, _I64, _PTR],
    "omni_window_attention": [_PTR, _I64, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_float,
                              _PTR, _PTR, _I64, _PTR, _PTR, _INT, _I64, _PTR, _I64, _PTR],
    "omni_silu_mul": [_PTR, _I64, _I64, _I64, _PTR, _I64, _PTR],
    "omni_dwconv_layernorm": [_PTR, _I64, _I64, _I64, _I64, _PTR, _PTR, _PTR, _PTR, ctypes.c_float,
                              _PTR, _I64, _PTR, _PTR, _I64, _INT, _PTR, _I64, _PTR],
    "omni_bias_gelu": [_PTR, _I64, _I64, _I64, _PTR, _PTR],
    "omni_bias_scale_residual": [_PTR, _I64, _I64, _PTR, _I64, _PTR, _PTR, _PTR, _I64, _PTR],
    "omni_advance_positions": [_PTR, _I64, _PTR, _I64, _I64, _INT, _PTR],
    "omni_gemm": [ctypes.POINTER(GemmArgs), _PTR],
    "omni_gemm_rope_kv": [ctypes.POINTER(GemmArgs), _I64, _I64, _I64, _I64, _PTR, _PTR, _PTR, _INT,
                          _I64, _PTR, _PTR, _I64, _PTR],
    "omni_resblock_pair": [ctypes.POINTER(ConvArgs), ctypes.POINTER(ConvArgs), _PTR],
    "omni_channel_embedding_sum": [_PTR, _INT, _I64, _I64, _I64, _I64, _PTR, _PTR, _INT, _I64, _PTR,
                                   _PTR],
}
_RESTYPES = {"omni_codec_error_string": ctypes.c_char_p}

_lib: ctypes.CDLL | None = None


def load_library(path: Path | str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and bind the native library; raises if it is absent or incomplete."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(path)
    if not path.exists():
        raise OmniCodecError(
            f"{path} is missing: build the HIP kernels first (python sglang-omni_amd/csrc/build.py)"
        )
    lib = ctypes.CDLL(str(path))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if a declared symbol is not exported
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != OK:
        msg = load_library().omni_codec_error_string(status).decode()
        raise OmniCodecError(f"{what}: status {status} ({msg})", status)


def require_device(*tensors: torch.Tensor) -> None:
    """The kernels run on the GPU only: refuse CPU tensors instead of falling back."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise OmniCodecError(
                f"the HIP codec kernels need GPU tensors; got a tensor on {t.device}"
            )


def require_vector(t: torch.Tensor | None, n: int, what: str, device: torch.device) -> None:
    """A per-channel coefficient array the kernels index up to n - 1: float32, contiguous, on
    the call's GPU, at least n entries."""
    if t is None:
        return
    require_device(t)
    if t.device != device:
        raise ValueError(f"{what} is on {t.device}, the call on {device}")
    if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() < n:
        raise ValueError(f"{what} must be contiguous float32 with at least {n} entries")


def require_slot_state(history: torch.Tensor | None, slot_index: torch.Tensor | None,
                       slot_parity: torch.Tensor | None, *, rows: int, samples: int,
                       channels: int, device: torch.device, what: str,
                       dtype: torch.dtype = torch.bfloat16) -> None:
    """A streaming history pool of `slots` contiguous slots, each holding at least two copies of
    [samples, channels] (e.g. [slots, 2, samples, channels]), with the int64 slot index of the
    call's rows and the pool's per-slot parity, all on the call's GPU: the kernels read
    slot_index[0 .. rows-1] and slot_parity[0 .. slots-1] as device arrays."""
    if history is None:
        return
    if slot_index is None or slot_parity is None:
        raise ValueError(f"{what}: a history pool needs slot_index and slot_parity")
    require_device(history, slot_index, slot_parity)
    for t, name in ((history, "history"), (slot_index, "slot_index"), (slot_parity, "slot_parity")):
        if t.device != device:
            raise ValueError(f"{what}: {name} is on {t.device}, the call on {device}")
    slots = history.shape[0] if history.dim() else 0
    if (history.dtype != dtype or history.dim() < 2 or slots < 1 or not history.is_contiguous()
            or history.numel() // slots < 2 * samples * channels):
        raise ValueError(f"{what}: history must be a contiguous {dtype} pool of slots holding "
                         f"2 x {samples} x {channels} elements each")
    if slot_index.dtype != torch.int64 or slot_index.dim() != 1 or slot_index.shape[0] < rows \
            or slot_index.stride(0) != 1:
        raise ValueError(f"{what}: slot_index must be contiguous int64 with {rows} entries")
    if slot_parity.dtype != torch.int64 or slot_parity.dim() != 1 \
            or slot_parity.shape[0] < slots or slot_parity.stride(0) != 1:
        raise ValueError(f"{what}: slot_parity must be contiguous int64 with an entry per slot")


def stream_handle(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def omni_dtype(dtype: torch.dtype) -> int:
    try:
        return TORCH_TO_OMNI[dtype]
    except KeyError:
        raise OmniCodecError(f"dtype {dtype} has no kernel") from None


def capabilities(device: int = 0) -> dict[str, object]:
    lib = load_library()
    arch = ctypes.create_string_buffer(64)
    lds = _I64()
    cus = _I64()
    check(lib.omni_codec_capabilities(device, arch, 64, ctypes.byref(lds), ctypes.byref(cus)),
          "omni_codec_capabilities")
    return {"arch": arch.value.decode(), "lds_bytes": lds.value, "compute_units": cus.value}
