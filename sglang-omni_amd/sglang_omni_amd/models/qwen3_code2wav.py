"""The Qwen3-Omni code2wav decoder on HIP kernels: ``forward`` / ``from_indices`` and streaming
slot decodes.

Drop-in for ``Qwen3OmniCode2Wav`` and ``Qwen3OmniIncrementalCodec.decode_slots``
(sglang_omni/models/qwen3_omni/components/code2wav.py:107-460) with a slot pool shaped as the
reference's ``CodecStatePool`` (codec_state_pool.py:26-145: conv histories, per-layer K/V rings
indexed ``slot * ring_frames + position % ring_frames``, frame positions). Weights are read by
``Qwen3OmniMoeCode2Wav.state_dict()`` names.

A decode step on channels-last activations:

    rvq_gather_sum (mean form)            codes -> h (float32 residual stream)
    per layer (8):
      rms_norm_residual                   h -> normed (bf16)
      GEMM qkv, rotary epilogue           normed -> qkv, q and k rotated at their positions;
                                          the new K / V rows into the rings
      window_attention                    q over the 72-frame window -> attn
      GEMM o, scaled residual epilogue    h += scale * (attn @ W_o^T)
      rms_norm_residual                   normed = RMSNorm(h)
      GEMM gate_up, silu_mul epilogue     normed -> act = silu(gate) * up
      GEMM down, scaled residual epilogue h += scale * (act @ W_down^T)
      rms_norm_residual                   normed = RMSNorm(h) (next layer / final)
    per upsampler (x2, x2):
      conv_dma (transposed, k = s)        normed -> r (float32, bias included)
      dwconv_layernorm                    r -> n (bf16; depthwise causal k7 with slot history)
      GEMM pwconv1, GELU epilogue         n -> p (bf16)
      GEMM pwconv2, scaled residual epilogue
                                          the next operand r + gamma * (p @ W2^T + b2) (bf16)
    the causal conv stack of ``DacCodecDecoder`` with SnakeBeta coefficients, transposed convs
    trimmed on both sides and the final clamp.

The GEMMs run on ``omni_gemm`` (kernels/gemm.py): bf16 operands, float32 accumulation over the
input features in one fixed order whatever the row count, the elementwise pass after each GEMM
on the accumulators. So a stream decoded in chunks gives the bits of its whole decode.
"""

from __future__ import annotations

import math
from typing import Any

import torch

from ..kernels import code2wav_front as F
from ..kernels.conv import fused_conv, pack_conv1d, pack_conv_transpose1d
from ..kernels.gemm import GELU, SCALED_RESIDUAL, linear, linear_rope_kv, pack_linear
from ..kernels.rvq import rvq_gather_sum
from .configs import Qwen3Code2WavConfig, Qwen3TTSCodecConfig
from .dac_codec import CodecStatePool, DacCodecDecoder, _Workspace

LN_EPS = 1e-6  # Qwen3OmniMoeConvNeXtBlock's LayerNorm


def conv_stack_tree(state: dict[str, torch.Tensor], config: Qwen3Code2WavConfig) -> dict[str, Any]:
    """The decoder convs of a code2wav state dict as ``DacCodecDecoder``'s weight tree, each
    SnakeBeta as its {"alpha", "beta"} log-parameters."""

    def conv(prefix: str) -> dict[str, torch.Tensor]:
        return {"weight": state[f"{prefix}.weight"].float(), "bias": state[f"{prefix}.bias"].float()}

    def snake(prefix: str) -> dict[str, torch.Tensor]:
        return {"alpha": state[f"{prefix}.alpha"].float(), "beta": state[f"{prefix}.beta"].float()}

    tree: dict[str, Any] = {"in_conv": conv("decoder.0.conv"), "blocks": []}
    for bi, rate in enumerate(config.upsample_rates, start=1):
        p = f"decoder.{bi}.block"
        tree["blocks"].append({
            "stride": rate,
            "alpha": snake(f"{p}.0"),
            "up": conv(f"{p}.1.conv"),
            "units": [{"dilation": d, "alpha1": snake(f"{p}.{u + 2}.act1"),
                       "conv1": conv(f"{p}.{u + 2}.conv1.conv"),
                       "alpha2": snake(f"{p}.{u + 2}.act2"),
                       "conv2": conv(f"{p}.{u + 2}.conv2.conv")}
                      for u, d in enumerate(config.dilations)],
        })
    n = len(config.upsample_rates)
    tree["final"] = {"alpha": snake(f"decoder.{n + 1}"), "conv": conv(f"decoder.{n + 2}.conv")}
    return tree


class Code2WavStatePool(CodecStatePool):
    """The conv stack's per-slot histories (``CodecStatePool``), plus what the front streams:
    per-layer K / V rings [slots * ring_frames, kv_heads * head_dim] bf16, the slots' frame
    positions, and the ConvNeXt depthwise convs' float32 histories [slots, 2, 6, C]."""

    def __init__(self, layout: list[tuple[str, int, int]], *, num_slots: int, capture_slots: int,
                 device: torch.device, num_layers: int, kv_width: int, ring_frames: int,
                 retained_frames: int, dw_names: list[str], channels: int):
        super().__init__(layout, num_slots=num_slots, capture_slots=capture_slots, device=device)
        if ring_frames <= retained_frames:
            raise ValueError("a ring holds the window and the new frames")
        total = num_slots + capture_slots
        self.ring_frames = ring_frames
        self.retained_frames = retained_frames
        self.keys = [torch.zeros(total * ring_frames, kv_width, dtype=torch.bfloat16, device=device)
                     for _ in range(num_layers)]
        self.values = [torch.zeros_like(ring) for ring in self.keys]
        self.frame_positions = torch.zeros(total, dtype=torch.int64, device=device)
        self.dw_histories = {name: torch.zeros(total, 2, 6, channels, dtype=torch.float32,
                                               device=device) for name in dw_names}
        self.bytes_per_slot += (2 * num_layers * ring_frames * kv_width * 2
                                + len(dw_names) * 2 * 6 * channels * 4 + 8)

    def zero_slots(self, slots: torch.Tensor) -> None:
        super().zero_slots(slots)
        for ring in (*self.keys, *self.values):
            ring.view(-1, self.ring_frames, ring.shape[1]).index_fill_(0, slots, 0)
        for pool in self.dw_histories.values():
            pool.index_fill_(0, slots, 0)
        self.frame_positions.index_fill_(0, slots, 0)


class Qwen3Code2WavDecoder(DacCodecDecoder):
    """Qwen3-Omni code2wav on gfx950 HIP kernels (the transformer's and ConvNeXt's GEMMs as k = 1
    convs on the LDS-DMA conv kernel). ``state`` is a
    ``Qwen3OmniMoeCode2Wav.state_dict()``-named float32 dict (``configs.make_qwen3_code2wav_
    weights``); conv weights are bf16 (``weight_format`` "fp8" quantizes the decoder convs)."""

    DEFAULT_RING_EXTRA = 64  # frames one decode may add to a pool built with the default ring

    def __init__(self, state: dict[str, torch.Tensor], config: Qwen3Code2WavConfig, *,
                 device: torch.device | str = "cuda", weight_format: str = "bf16",
                 residual_stacks: bool = True, residual_dtype: torch.dtype = torch.float16):
        super().__init__(conv_stack_tree(state, config), config, device=device,
                         weight_format=weight_format, residual_stacks=residual_stacks,
                         residual_dtype=residual_dtype)
        cfg = config
        dev = self.device
        if cfg.head_dim != 64:
            raise ValueError("the attention kernel takes head_dim 64")
        self.front_upsample = int(math.prod(cfg.upsampling_ratios))
        self.num_codebooks = cfg.num_quantizers
        c = cfg.hidden_size
        self.hidden = c
        # the transformer's input / output width (Qwen3-TTS projects from / to latent_dim)
        self.latent = getattr(cfg, "latent_dim", c)
        self.q_width = cfg.num_attention_heads * cfg.head_dim
        self.kv_width = cfg.num_key_value_heads * cfg.head_dim
        self.split_rvq = hasattr(cfg, "semantic_quantizers")

        def bf16(t: torch.Tensor) -> torch.Tensor:
            return t.float().to(torch.bfloat16).to(dev).contiguous()

        def f32(t: torch.Tensor) -> torch.Tensor:
            return t.float().to(dev).contiguous()

        self.pre_conv = self.input_proj = self.output_proj = None
        if self.split_rvq:
            # each codebook's entries projected by its group's output projection once, so the
            # dequantize is one gather-sum: sum_k (W_g(k) E_k)[code_k]
            books = state["quantizer.codebooks"].double()
            sem = state["quantizer.semantic_proj.weight"].double()
            aco = state["quantizer.acoustic_proj.weight"].double()
            proj = [books[k] @ (sem if k < cfg.semantic_quantizers else aco).t()
                    for k in range(cfg.num_quantizers)]
            self.code_tables = torch.stack(proj).float().to(dev).contiguous()
            self.pre_conv = pack_conv1d(state["pre_conv.conv.weight"].float(),
                                        state["pre_conv.conv.bias"].float()).to(dev)
            self.input_proj = pack_conv1d(
                state["pre_transformer.input_proj.weight"].float()[..., None],
                state["pre_transformer.input_proj.bias"].float()).to(dev)
            self.output_proj = pack_conv1d(
                state["pre_transformer.output_proj.weight"].float()[..., None],
                state["pre_transformer.output_proj.bias"].float()).to(dev)
        else:
            self.code_tables = bf16(state["code_embedding.weight"].view(cfg.num_quantizers,
                                                                        cfg.codebook_size, c))
        self.layers = []
        for i in range(cfg.num_hidden_layers):
            p = f"pre_transformer.layers.{i}"
            qkv = torch.cat([state[f"{p}.self_attn.{n}_proj.weight"] for n in "qkv"], dim=0)
            gate_up = torch.cat([state[f"{p}.mlp.gate_proj.weight"],
                                 state[f"{p}.mlp.up_proj.weight"]], dim=0)
            # GEMM weights [out, in] as bf16 rows (gate / up interleaved for the silu epilogue)
            self.layers.append({
                "in_norm": f32(state[f"{p}.input_layernorm.weight"]),
                "qkv": pack_linear(qkv).to(dev),
                "o": pack_linear(state[f"{p}.self_attn.o_proj.weight"]).to(dev),
                "attn_scale": f32(state[f"{p}.self_attn_layer_scale.scale"]),
                "post_norm": f32(state[f"{p}.post_attention_layernorm.weight"]),
                "gate_up": pack_linear(gate_up, gated=True).to(dev),
                "down": pack_linear(state[f"{p}.mlp.down_proj.weight"]).to(dev),
                "mlp_scale": f32(state[f"{p}.mlp_layer_scale.scale"]),
            })
        self.final_norm = f32(state["pre_transformer.norm.weight"])
        # inv_freq as the rotary module computes it, in float32
        self.inv_freq = (1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2,
                                                                dtype=torch.float32)
                                                   / cfg.head_dim))).to(dev).contiguous()
        # one launch for the qkv GEMM and the rotary embedding where a wave's 64 columns are one
        # head (64-wide heads, q + k + v columns a multiple of 128); else two, with the same bits
        qkv_cols = (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim
        self.fused_rope = cfg.head_dim == 64 and qkv_cols % 128 == 0
        self.upsamplers = []
        for i, factor in enumerate(cfg.upsampling_ratios):
            p = f"upsample.{i}.1"
            self.upsamplers.append({
                "name": f"upsample.{i}.convnext.dwconv",
                "factor": factor,
                "up": pack_conv_transpose1d(state[f"upsample.{i}.0.conv.weight"].float(),
                                            state[f"upsample.{i}.0.conv.bias"].float(),
                                            stride=factor).to(dev),
                "dw_weight": f32(state[f"{p}.dwconv.conv.weight"][:, 0, :].t()),  # [7, C]
                "dw_bias": f32(state[f"{p}.dwconv.conv.bias"]),
                "ln_weight": f32(state[f"{p}.norm.weight"]),
                "ln_bias": f32(state[f"{p}.norm.bias"]),
                "w1": pack_linear(state[f"{p}.pwconv1.weight"],
                                  state[f"{p}.pwconv1.bias"]).to(dev),
                "w2": pack_linear(state[f"{p}.pwconv2.weight"],
                                  state[f"{p}.pwconv2.bias"]).to(dev),
                "gamma": f32(state[f"{p}.gamma"]),
            })
            if self.upsamplers[-1]["up"].taps != 1:
                raise ValueError("the upsamplers' transposed convs have k = s")

    # ---------------------------------------------------------------- state pool

    def state_layout(self) -> list[tuple[str, int, int]]:
        layout = super().state_layout()
        if self.pre_conv is not None:
            layout.insert(0, ("pre_conv", self.latent, self.pre_conv.left_pad))
        return layout

    def new_state_pool(self, num_slots: int, capture_slots: int = 0,
                       ring_frames: int | None = None) -> Code2WavStatePool:
        """A pool whose rings hold the window and up to ``ring_frames - (sliding_window - 1)``
        new frames per decode (default: 64)."""
        retained = self.config.sliding_window - 1
        if ring_frames is None:
            ring_frames = retained + self.DEFAULT_RING_EXTRA
        return Code2WavStatePool(
            self.state_layout(), num_slots=num_slots, capture_slots=capture_slots,
            device=self.device, num_layers=self.config.num_hidden_layers,
            kv_width=self.kv_width, ring_frames=ring_frames, retained_frames=retained,
            dw_names=[u["name"] for u in self.upsamplers], channels=self.latent)

    # ---------------------------------------------------------------- front

    def _front_buffers(self, ws: _Workspace, batch: int, frames: int) -> dict[str, torch.Tensor]:
        if ws.front:
            return ws.front
        dev, c, cfg = self.device, self.hidden, self.config
        u = self.latent
        m = batch * frames
        bf = torch.bfloat16
        width = self.q_width + 2 * self.kv_width
        buf = {
            "h": torch.empty(m, c, dtype=torch.float32, device=dev),
            "normed": torch.empty(m, c, dtype=bf, device=dev),
            "qkv": torch.empty(m, width, dtype=bf, device=dev),
            "attn": torch.empty(m, self.q_width, dtype=bf, device=dev),
            "act": torch.empty(m, cfg.intermediate_size, dtype=bf, device=dev),
        }
        if self.split_rvq:
            buf["quantized"] = torch.empty(batch, frames, u, dtype=bf, device=dev)
            buf["pre"] = torch.empty(batch, frames, u, dtype=bf, device=dev)
            buf["latent"] = torch.empty(batch, frames, u, dtype=bf, device=dev)
        length = frames
        for i, up in enumerate(self.upsamplers):
            length *= up["factor"]
            buf[f"r{i}"] = torch.empty(batch, length, u, dtype=torch.float32, device=dev)
            buf[f"n{i}"] = torch.empty(batch, length, u, dtype=bf, device=dev)
            buf[f"p1_{i}"] = torch.empty(batch * length, up["w1"].out_features, dtype=bf,
                                          device=dev)
            buf[f"z{i}"] = torch.empty(batch, length, u, dtype=bf, device=dev)
        ws.front.update(buf)
        return ws.front

    def _front(self, codes: torch.Tensor, ws: _Workspace,
               state: dict | None) -> tuple[torch.Tensor, int]:
        cfg = self.config
        batch, books, frames = codes.shape
        if books != cfg.num_quantizers:
            raise ValueError(f"Expected {cfg.num_quantizers} layer of codes, got {books}")
        buf = self._front_buffers(ws, batch, frames)
        timer = self.timer
        c, m = self.hidden, batch * frames
        pool = None if state is None else state["pool"]
        cold = True if state is None else bool(state["cold"])
        slots = None if state is None else state["slot_index"]
        if state is not None:
            state["new_frames"] = frames
            if not cold and frames > pool.ring_frames - pool.retained_frames:
                raise ValueError(f"{frames} new frames overflow the pool's {pool.ring_frames}-frame "
                                 f"rings (window {pool.retained_frames} + new frames)")
        h, normed, qkv = buf["h"], buf["normed"], buf["qkv"]
        attn, act = buf["attn"], buf["act"]
        k_books, _, dim = self.code_tables.shape
        tab = self.code_tables.element_size()
        with timer.launch("rvq", m * (k_books * dim * tab + dim * 4 + k_books * codes.element_size())):
            if self.split_rvq:
                rvq_gather_sum(codes, self.code_tables, out=buf["quantized"], clamp=True)
            else:
                rvq_gather_sum(codes, self.code_tables, out=h.view(batch, frames, c), mean=True,
                               clamp=True)
        if self.split_rvq:
            # causal pre_conv (its context from the slot history), then input_proj (+ bias)
            # into the float32 residual stream
            pc = self.pre_conv
            hist = {}
            if pool is not None:
                hist = {"history": pool.histories.get("pre_conv"), "slot_index": slots,
                        "slot_parity": pool.parity, "history_cold": cold}
            with timer.launch("conv", 2.0 * m * pc.macs_per_position, "pre_conv"):
                fused_conv(buf["quantized"], pc, buf["pre"], **hist)
            ip = self.input_proj
            with timer.launch("conv", 2.0 * m * ip.macs_per_position, "input_proj"):
                fused_conv(buf["pre"], ip, None, sum_out=h.view(batch, frames, c))
        heads, kv_heads, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        eps = cfg.rms_norm_eps
        with timer.launch("front_elementwise", 0.0):
            F.rms_norm_residual(h, self.layers[0]["in_norm"], eps, normed)
        for i, layer in enumerate(self.layers):
            ring = {}
            if pool is not None:
                ring = {"slot_index": slots, "positions": pool.frame_positions,
                        "key_ring": pool.keys[i], "value_ring": pool.values[i],
                        "ring_frames": pool.ring_frames}
            if self.fused_rope:
                # the rotary embedding and the K / V ring writes in the qkv GEMM's epilogue
                with timer.launch("front_gemm", 2.0 * m * c * qkv.shape[1]):
                    linear_rope_kv(normed, layer["qkv"], qkv, batch, heads, kv_heads, hd,
                                   self.inv_freq, cold=cold, **ring)
            else:
                with timer.launch("front_gemm", 2.0 * m * c * qkv.shape[1]):
                    linear(normed, layer["qkv"], qkv)
                with timer.launch("front_elementwise", 0.0):
                    F.rope_kv_write(qkv, batch, heads, kv_heads, hd, self.inv_freq, cold=cold,
                                    **ring)
            # a first decode attends to its own frames: the keys are in qkv already
            attend_ring = {} if cold else ring
            with timer.launch("front_attention", 4.0 * m * heads * hd * cfg.sliding_window):
                F.window_attention(qkv, batch, heads, kv_heads, hd, cfg.sliding_window,
                                   hd ** -0.5, attn, cold=cold, **attend_ring)
            # h += attn_scale * o(attn), mlp likewise: the scaled residual in the GEMM epilogue
            with timer.launch("front_gemm", 2.0 * m * self.q_width * c):
                linear(attn, layer["o"], h, epilogue=SCALED_RESIDUAL, scale=layer["attn_scale"],
                       residual=h)
            with timer.launch("front_elementwise", 0.0):
                F.rms_norm_residual(h, layer["post_norm"], eps, normed)
            with timer.launch("front_gemm", 2.0 * m * c * 2 * act.shape[1]):
                linear(normed, layer["gate_up"], act)
            with timer.launch("front_gemm", 2.0 * m * act.shape[1] * c):
                linear(act, layer["down"], h, epilogue=SCALED_RESIDUAL, scale=layer["mlp_scale"],
                       residual=h)
            nxt = self.layers[i + 1]["in_norm"] if i + 1 < len(self.layers) else self.final_norm
            with timer.launch("front_elementwise", 0.0):
                F.rms_norm_residual(h, nxt, eps, normed)
        x = normed.view(batch, frames, c)
        if self.output_proj is not None:
            op = self.output_proj
            with timer.launch("conv", 2.0 * m * op.macs_per_position, "output_proj"):
                fused_conv(x, op, buf["latent"])
            x = buf["latent"]
        length = frames
        for i, up in enumerate(self.upsamplers):
            factor = up["factor"]
            r = buf[f"r{i}"]
            with timer.launch("conv", 2.0 * batch * length * up["up"].macs_per_position,
                              f"upsample.{i}.up"):
                fused_conv(x, up["up"], None,
                           sum_out=r.view(batch, length, factor * self.latent))
            length *= factor
            hist = {}
            if pool is not None:
                hist = {"history": pool.dw_histories[up["name"]], "slot_index": slots,
                        "slot_parity": pool.parity, "history_cold": cold}
            n = buf[f"n{i}"]
            with timer.launch("front_elementwise", 0.0):
                F.dwconv_layernorm(r, up["dw_weight"], up["dw_bias"], up["ln_weight"],
                                   up["ln_bias"], LN_EPS, n, **hist)
            rows = batch * length
            u = self.latent
            p1 = buf[f"p1_{i}"]
            with timer.launch("front_gemm", 2.0 * rows * u * p1.shape[1]):
                linear(n.view(rows, u), up["w1"], p1, epilogue=GELU)
            # the next operand r + gamma * (pwconv2(p1) + b2), rounded once to bf16
            z = buf[f"z{i}"]
            with timer.launch("front_gemm", 2.0 * rows * p1.shape[1] * u):
                linear(p1, up["w2"], z.view(rows, u), epilogue=SCALED_RESIDUAL,
                       scale=up["gamma"], residual=r.view(rows, u))
            x = z
        return x, length

    def _finish_step(self, wave: torch.Tensor, state: dict | None, batch: int) -> torch.Tensor:
        if state is not None:
            F.advance_positions(state["pool"].frame_positions, state["slot_index"],
                                state["new_frames"], bool(state["cold"]))
        return super()._finish_step(wave, state, batch)

    # ---------------------------------------------------------------- API

    @torch.no_grad()
    def from_indices(self, indices: torch.Tensor) -> torch.Tensor:
        """Qwen3OmniMoeCode2Wav.forward: [B, Q, T] codes -> [B, 1, samples] float32 (the whole
        decode drops each decoder transposed conv's first and last s samples). Long inputs
        decode in chunks through a temporary slot pool, which gives the same samples."""
        if indices.dim() != 3:
            raise ValueError(f"codes must be [B, Q, T], got {tuple(indices.shape)}")
        batch, _, frames = indices.shape
        step = self.frames_per_call(batch)
        if frames <= step:
            return self._decode(indices, None)
        pool = self.new_state_pool(num_slots=batch,
                                   ring_frames=self.config.sliding_window - 1 + step)
        rows = torch.arange(batch, device=self.device)
        parts = [self._decode(indices[..., s:s + step],
                              {"pool": pool, "slot_index": rows, "cold": s == 0})
                 for s in range(0, frames, step)]
        return torch.cat(parts, dim=-1)

    __call__ = from_indices
    forward = from_indices


class Qwen3TTSCodecState:
    """One cohort of streams' decoder state for ``Qwen3TTSCodecDecoder.decode``, as the
    reference's ``Qwen3TTSIncrementalCodecState`` (qwen3_tts/incremental_codec.py:74-133)
    carries it: rows bound to slots of a slot pool (conv histories, transposed-conv contexts,
    K / V rings, the slots' frame positions).

    * ``init_state``: a private pool with one slot per row; every row starts together and
      ``frame_position`` counts the frames they have decoded (the first decode is cold).
    * ``Qwen3TTSCodecStateArena.gather``: rows bound to arena slots in place (no copy); each
      slot carries its own absolute position (``frame_positions``, settable), and a fresh slot
      is zeroed, so cold and warm rows decode together.
    """

    def __init__(self, pool: Code2WavStatePool, batch_size: int, device: torch.device, *,
                 slot_index: torch.Tensor | None = None, per_row_positions: bool = False):
        self.pool = pool
        self.batch_size = batch_size
        self.slot_index = (torch.arange(batch_size, dtype=torch.int64, device=device)
                           if slot_index is None else slot_index)
        self.frame_position = 0
        self.per_row_positions = per_row_positions
        self.slots: list[int] | None = None  # the host slot ids of an arena cohort

    @property
    def frame_positions(self) -> torch.Tensor:
        """The rows' absolute frame positions (on the device)."""
        return self.pool.frame_positions[self.slot_index]

    @frame_positions.setter
    def frame_positions(self, positions) -> None:
        values = torch.as_tensor(positions, dtype=torch.int64)
        if values.shape != (self.batch_size,):
            raise ValueError(f"{self.batch_size} rows, {tuple(values.shape)} positions")
        self.pool.frame_positions.index_copy_(0, self.slot_index,
                                              values.to(self.pool.frame_positions.device))

    def advance(self, fresh_frames: int) -> None:
        self.frame_position += fresh_frames


class Qwen3TTSCodecDecoder(Qwen3Code2WavDecoder):
    """The Qwen3-TTS tokenizer's decoder with the reference's incremental API
    (``Qwen3TTSIncrementalDecoder``, qwen3_tts/incremental_codec.py:771-1083): ``init_state``
    and ``decode(codes, state)``, every decode of T fresh frames emitting T * total_upsample
    samples and advancing the state in place; the rows of a state decode together."""

    def __init__(self, state: dict[str, torch.Tensor], config: Qwen3TTSCodecConfig, *,
                 device: torch.device | str = "cuda", weight_format: str = "bf16",
                 residual_stacks: bool = True, residual_dtype: torch.dtype = torch.float16):
        if getattr(config, "transconv_trim", "right") != "right":
            raise ValueError("the Qwen3-TTS decoder trims its transposed convs on the right")
        super().__init__(state, config, device=device, weight_format=weight_format,
                         residual_stacks=residual_stacks, residual_dtype=residual_dtype)
        self.total_upsample = config.hop_length
        self.compiled_shapes: set[tuple[int, int]] = set()

    def init_state(self, batch_size: int, *, device: torch.device | None = None,
                   max_fresh_frames: int | None = None) -> Qwen3TTSCodecState:
        """A zeroed state for ``batch_size`` rows whose decodes take at most
        ``max_fresh_frames`` frames (default 64)."""
        if batch_size < 1:
            raise ValueError("a state holds at least one row")
        retained = self.config.sliding_window - 1
        extra = self.DEFAULT_RING_EXTRA if max_fresh_frames is None else max_fresh_frames
        pool = self.new_state_pool(num_slots=batch_size, ring_frames=retained + extra)
        return Qwen3TTSCodecState(pool, batch_size, device or self.device)

    def decode(self, codes: torch.Tensor, state: Qwen3TTSCodecState, *,
               compiled: bool = False) -> torch.Tensor:
        """(B, Q, T) codes after the frames ``state`` holds -> (B, 1, T * total_upsample)
        waveform; ``state`` advances by T frames."""
        if codes.ndim != 3:
            raise ValueError("Qwen3-TTS incremental codec decoding requires codes shaped [B, Q, T]")
        if int(codes.shape[0]) < 1:
            raise ValueError("Qwen3-TTS incremental codec decoding requires at least one row")
        fresh_frames = int(codes.shape[-1])
        if fresh_frames <= 0:
            raise ValueError("Qwen3-TTS incremental codec decoding requires fresh frames")
        shape = (int(codes.shape[0]), fresh_frames)
        if compiled and shape not in self.compiled_shapes:
            raise RuntimeError(f"Qwen3-TTS incremental codec shape {shape} was not precompiled")
        if int(codes.shape[0]) != state.batch_size:
            raise ValueError(f"the state holds {state.batch_size} rows, the codes {codes.shape[0]}")
        with torch.no_grad():
            waveform = self._decode(codes, self._step_state(state))
        if int(waveform.shape[-1]) != fresh_frames * self.total_upsample:
            raise RuntimeError("Qwen3-TTS incremental codec decoder returned the wrong sample count")
        state.advance(fresh_frames)
        return waveform

    @staticmethod
    def _step_state(state: Qwen3TTSCodecState) -> dict:
        # arena rows decode warm: a fresh slot is zeroed (histories, contexts, K / V, position
        # 0), which is what a cold decode reads, and the attention keys start at position 0
        cold = not state.per_row_positions and state.frame_position == 0
        return {"pool": state.pool, "slot_index": state.slot_index, "cold": cold}

    def tail_frames(self, emit_frames: int) -> int:
        """The code frames the last ``emit_frames`` frames' samples and the conv stack's state
        depend on (``tail_frames``, qwen3_tts/incremental_codec.py:1085-1110), walked back from
        the waveform: a causal conv adds its context, a transposed conv of kernel k and stride s
        maps n samples to (n + k - 1) // s inputs."""
        samples = int(emit_frames) * self.total_upsample + (self.final_taps - 1)
        for blk in reversed(self.blocks):
            for unit in reversed(blk.units):
                samples += unit.conv1.conv.left_pad  # the k = 1 conv adds none
            samples = (samples + blk.up_kernel - 1) // blk.stride
        samples += self.in_conv.conv.left_pad
        for up in reversed(self.upsamplers):
            samples += up["dw_weight"].shape[0] - 1  # the ConvNeXt depthwise conv
            samples = (samples + up["factor"] - 1) // up["factor"]  # kernel = stride
        return samples

    def decode_tail(self, codes: torch.Tensor, valid_frames, state: Qwen3TTSCodecState,
                    emit_frames: int) -> torch.Tensor:
        """Row i's first ``valid_frames[i]`` frames of ``codes`` decoded after its state, the
        conv stack run over the last ``tail_frames(emit_frames)`` of them only; returns the
        samples of the last ``emit_frames`` frames of each row, (B, 1, emit_frames * hop), and
        advances each row by its valid frames (``decode_tail``, qwen3_tts/incremental_codec.py:
        1112-1134). Needs arena rows (per-row positions) and tail_frames <= valid_frames[i] <=
        T. Rows of one width decode together (their transformer, pre_conv and ConvNeXt state
        end at their own last frame)."""
        if not state.per_row_positions:
            raise ValueError("Qwen3-TTS tail decoding needs per-row frame positions")
        if codes.ndim != 3 or int(codes.shape[0]) != state.batch_size:
            raise ValueError(f"codes must be [{state.batch_size}, Q, T], got {tuple(codes.shape)}")
        widths = [int(w) for w in torch.as_tensor(valid_frames).reshape(-1).tolist()]
        if len(widths) != state.batch_size:
            raise ValueError(f"{len(widths)} valid frame counts for {state.batch_size} rows")
        tail = self.tail_frames(emit_frames)
        if emit_frames < 1 or any(w < tail or w > codes.shape[-1] for w in widths):
            raise ValueError(f"every row needs between tail_frames ({tail}) and {codes.shape[-1]} "
                             f"valid frames, and emit_frames >= 1; got {widths}")
        samples = int(emit_frames) * self.total_upsample
        out = torch.empty(state.batch_size, 1, samples, dtype=torch.float32, device=self.device)
        with torch.no_grad():
            for w in sorted(set(widths)):
                rows = [i for i, v in enumerate(widths) if v == w]
                if len(rows) == state.batch_size:
                    sub_codes, sub_index = codes[..., :w], state.slot_index
                else:
                    pick = torch.tensor(rows, dtype=torch.int64).to(self.device)
                    sub_codes = codes.index_select(0, pick)[..., :w]
                    sub_index = state.slot_index.index_select(0, pick)
                step = {"pool": state.pool, "slot_index": sub_index, "cold": False}
                wave = self._decode(sub_codes.contiguous(), step, window=tail)
                if len(rows) == state.batch_size:
                    out.copy_(wave[..., -samples:])
                else:
                    out.index_copy_(0, pick, wave[..., -samples:].contiguous())
        return out



    def precompile(self, codes: torch.Tensor, state: Qwen3TTSCodecState) -> None:
        """Admit (B, T) for ``decode(..., compiled=True)``: the HIP path needs no tracing, so this
        records the shape and, as the reference's precompile does, runs (and advances) one
        decode."""
        shape = (int(codes.shape[0]), int(codes.shape[-1]))
        self.compiled_shapes.add(shape)
        self.decode(codes, state)
