"""Write the golden fixtures of the codec decode path from the float32 oracle.

Each fixture holds the seeded inputs that are small enough to keep (codes, mel frames), a SHA-256
of the inputs regenerated from their seeds (tables, conv weights), and the oracle's outputs.
tests/test_golden.py regenerates the inputs, checks the digests (a change in torch's generator
would show there first) and compares the oracle and, on the GPU, the HIP path with the stored
outputs.

    python tests/golden/make_golden.py        # rewrites tests/golden/*.npz
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
for _p in (REPO / "sglang-omni_amd", REPO):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

from oracle import codec_oracle as O  # noqa: E402
from sglang_omni_amd.models.configs import (  # noqa: E402
    DacDecoderConfig,
    HifiGanConfig,
    make_dac_weights,
    make_hifigan_weights,
)
from sglang_omni_amd.quantization import reference_weights  # noqa: E402

TINY_DAC = DacDecoderConfig(n_codebooks=4, codebook_size=64, latent_dim=64, channels=128,
                            rates=(2, 4), conv_gain=0.85)
# gain 0.4: output RMS ~0.04, the level of the full-size vocoder (tanh's linear range)
TINY_HIFIGAN = HifiGanConfig(n_mels=16, channels=64, rates=(2, 3), up_kernels=(4, 7), conv_gain=0.4)


def digest(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().contiguous().cpu().numpy().tobytes())
    return h.hexdigest()


def tree_digest(tree) -> str:
    leaves = []

    def walk(node):
        if isinstance(node, torch.Tensor):
            leaves.append(node)
        elif isinstance(node, dict):
            for k in sorted(node):
                walk(node[k])
        elif isinstance(node, (list, tuple)):
            for v in node:
                walk(v)

    walk(tree)
    return digest(*leaves)


def single_block_inputs():
    """RVQ (K = 8 tables of 1024 x 256 ~ N(0, 0.02), int32 codes uniform in [0, 1024), T = 50)
    then causal Conv1d 256 -> 256 k = 7 (torch's default init) -> Snake(alpha = 1) -> + x, all
    drawn from torch.manual_seed(0) in this order."""
    torch.manual_seed(0)
    tables = torch.randn(8, 1024, 256) * 0.02
    codes = torch.randint(0, 1024, (1, 8, 50), dtype=torch.int32)
    conv = torch.nn.Conv1d(256, 256, 7)
    return tables, codes, conv.weight.detach(), conv.bias.detach(), torch.ones(256)


def tiny_dac_inputs():
    weights = make_dac_weights(TINY_DAC, seed=0)
    codes = torch.randint(0, 64, (3, 4, 17), generator=torch.Generator().manual_seed(1))
    return weights, codes


def tiny_hifigan_inputs():
    weights = make_hifigan_weights(TINY_HIFIGAN, seed=0)
    mel = torch.randn(2, 16, 10, generator=torch.Generator().manual_seed(0)) * 2 - 5
    return weights, mel


def main() -> None:
    torch.set_num_threads(1)
    tables, codes, w, b, alpha = single_block_inputs()
    x, y = O.conv_block(codes, tables, w, b, alpha)
    np.savez_compressed(HERE / "single_block.npz", codes=codes.numpy(), rvq=x.numpy(),
                        block=y.numpy(), inputs_sha256=np.array(digest(tables, w, b)))

    weights, codes = tiny_dac_inputs()
    wave = O.dac_from_indices(codes, reference_weights(weights, "bf16"))
    np.savez_compressed(HERE / "tiny_dac.npz", codes=codes.numpy(), waveform=wave.numpy(),
                        weights_sha256=np.array(tree_digest(weights)))

    weights, mel = tiny_hifigan_inputs()
    wave = O.hifigan_generator(mel, reference_weights(weights, "bf16"))
    np.savez_compressed(HERE / "tiny_hifigan.npz", mel=mel.numpy(), waveform=wave.numpy(),
                        weights_sha256=np.array(tree_digest(weights)))
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")


if __name__ == "__main__":
    main()
