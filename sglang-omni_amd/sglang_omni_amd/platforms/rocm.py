"""The ROCm / MI355X platform entry of the codec decode stage.

Counterpart of ``ROCMOmniPlatform`` (sglang_omni/platforms/rocm.py:22-131) for the vocoder hot
path: where the reference's ROCm entry turns the fast codec path off (code2wav graphs disabled,
rocm.py:130-131; channels-last convs CUDA-only, sglang_omni/utils/channels_last_conv.py:12-14),
this one reports the HIP kernels as the codec path and enables graph capture of decode steps.
"""

from __future__ import annotations

import os

import torch

from .. import _native as N


class ROCmCodecPlatform:
    device_name = "rocm"
    device_type = "cuda"  # HIP devices surface as torch's "cuda" device type
    required_arch = "gfx950"

    def is_rocm(self) -> bool:
        return torch.version.hip is not None

    def is_cuda(self) -> bool:
        return False

    def is_available(self) -> bool:
        return self.is_rocm() and torch.cuda.is_available()

    def enable_code2wav_graph(self) -> bool:
        """Every codec kernel is stream-ordered, allocation-free and host-sync-free, so decode
        steps may be captured (``SGLANG_OMNI_CODEC_GRAPHS=0`` turns it off)."""
        return os.environ.get("SGLANG_OMNI_CODEC_GRAPHS", "1") != "0"

    def get_device_graph_backend(self) -> str:
        return "hip_graph"

    def codec_capabilities(self, device: int = 0) -> dict[str, object]:
        """arch / LDS / CU count from the native library; raises if it is not gfx950."""
        caps = N.capabilities(device)
        if not str(caps["arch"]).startswith(self.required_arch):
            raise N.OmniCodecError(
                f"the codec kernels are built for {self.required_arch}, device is {caps['arch']}"
            )
        return caps


current_platform = ROCmCodecPlatform()
