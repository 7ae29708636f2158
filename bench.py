"""Benchmark of the codec decode stage on one MI355X.

Default workload (the streaming serving pattern): the 24 kHz codec decoder (16 x 2048 x 512 RVQ
tables, 1536 channels, strides 8/8/5/6 = x1920) decoding 64 independent streams; one step decodes
a 12-frame chunk of every stream (768 frames = 61.44 audio-seconds) with the per-layer causal-conv
state held in the HBM slot pool, 20 chunks per stream (the streams restart every 20 steps). Codes
are uniform random per stream (seed 1 + s), weights seeded random (kaiming, bf16). Inputs are
staged in HBM before the timed region.

Prints one JSON line: audio-seconds decoded per wall-second (xRT), plus
  roofline      the fused MFMA kernel with the largest share of the step (the residual stack of
                the 96-channel stage): algorithmic FLOPs per launch over its mean launch time,
                timed with HIP events on the launch stream;
  rvq_gather    the RVQ gather-sum's achieved bytes/s, in the step and on a large batch;
  cpu_baseline  the float32 CPU restatement of the reference path (oracle/codec_oracle.py) timed
                on this host's cores on a bounded sample of the same workload;
  other_configs the xRT of the other decoder configurations: the single 20 s utterance, the
                HiFiGAN mel vocoder (16 x 10 s) and the fp8-weight long form (8 x 120 s), with
                the same long form on bf16 weights beside it;
  hift_transforms  HiFT's source spectrum and fused iSTFT tail at the HiFiGAN size, in HBM GB/s;
  qwen3_code2wav the Qwen3-Omni code2wav (pre-transformer + ConvNeXt + decoder) streaming 64
                streams x 12-frame chunks, eager and HIP-graph replayed, per-kind kernel times;
  qwen3_tts_codec the Qwen3-TTS tokenizer decoder through decode(codes, state), 64 rows x 12
                frames per decode;
  egress        one step's waveform leaving the device: the PCM16 egress kernel (HBM GB/s) and
                the staging of the step through a pinned slot to host arrays (PCIe-inclusive);
  calibration   the box's practical peaks: a 1 GiB copy and a bf16 8192^3 GEMM.

--only qwen3_code2wav runs the Qwen3-Omni code2wav leg alone (its kernel-trace profile).
--only stack96 / --only copy run one kernel alone for hardware-counter profiles: the roofline
kernel (the 96-channel residual stack of the same decoder, x [64, 23040, 96]) or a plain 1 GiB
device copy (the calibration of the FETCH_SIZE / WRITE_SIZE counters), --launches times each.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO / "sglang-omni_amd", REPO):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import torch  # noqa: E402

METRIC = "audio-sec decoded per wall-sec (xRT) at batch 64; HBM GB/s & MFMA % of peak"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBPS = 8000.0
CHUNK_FRAMES = 12
CHUNKS_PER_STREAM = 20
STREAMS = 64


KERNEL_NAMES = {
    "stack96": "residual_stack_kernel, 96 channels: 3 residual units (conv k7 dilation 1/3/9 + "
               "Snake + conv k1 + residual) and the final conv 96->1 k7 + tanh per launch",
    "unit96": "conv_mfma_kernel fused residual unit, 96 channels (conv k7 + Snake + conv k1 + "
              "residual)",
    "unit192": "conv_mfma_kernel fused residual unit, 192 channels (conv k7 + Snake + conv k1 + "
               "residual)",
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def sync() -> None:
    torch.cuda.synchronize()


def timed_steps(step, steps: int, warmup: int) -> float:
    for i in range(warmup):
        step(i)
    sync()
    t0 = time.perf_counter()
    for i in range(steps):
        step(warmup + i)
    sync()
    return time.perf_counter() - t0


def measure_rvq_large(device: torch.device) -> dict:
    """The gather-sum alone at the long-form quantizer's shape: 8 x 1500 frames, 32 codebooks of
    1024 x 512 bf16, int32 codes, bf16 output (33 920 B per frame)."""
    from sglang_omni_amd.kernels.rvq import rvq_gather_sum

    gen = torch.Generator().manual_seed(0)
    tables = (torch.randn(32, 1024, 512, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    codes = torch.randint(0, 1024, (8, 32, 1500), generator=gen, dtype=torch.int32).to(device)
    out = torch.empty(8, 1500, 512, dtype=torch.bfloat16, device=device)
    frames = 8 * 1500
    per_frame = 32 * 512 * 2 + 512 * 2 + 32 * 4
    for _ in range(3):
        rvq_gather_sum(codes, tables, out=out)
    reps = 20
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        rvq_gather_sum(codes, tables, out=out)
    end.record()
    sync()
    ms = start.elapsed_time(end) / reps
    gbps = frames * per_frame / (ms * 1e-3) / 1e9
    return {"frames": frames, "bytes_per_frame": per_frame, "ms": round(ms, 4),
            "achieved_GBps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4)}


def cpu_baseline(config, weights, frames: int, streams: int) -> dict:
    """The float32 CPU restatement of the reference decode path on `streams` x `frames` frames."""
    from oracle import codec_oracle as O
    from sglang_omni_amd.quantization import reference_weights

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    ref = reference_weights(weights, "bf16")
    gen = torch.Generator().manual_seed(1)
    codes = torch.randint(0, config.codebook_size, (streams, config.n_codebooks, frames),
                          generator=gen)
    O.dac_from_indices(codes[:1, :, :2], ref)  # warm the CPU kernels
    t0 = time.perf_counter()
    with torch.no_grad():
        O.dac_from_indices(codes, ref)
    dt = time.perf_counter() - t0
    audio = streams * frames / config.frame_rate
    return {"value": round(audio / dt, 3), "unit": "audio-s/s", "cores": threads, "kind": "port",
            "sample": f"{streams} streams x {frames} frames ({audio:.2f} audio-s) whole-stream "
                      f"decode, float32, torch CPU, {dt:.1f} s"}


def bench_streaming(args, device) -> dict:
    from sglang_omni_amd.models import DacCodecDecoder, make_dac_weights
    from sglang_omni_amd.models.configs import CODEC_24K, dac_macs_per_frame
    from sglang_omni_amd.utils.timing import NO_TIMER, LaunchTimer

    config = CODEC_24K
    weights = make_dac_weights(config, seed=0)
    decoder = DacCodecDecoder(weights, config, device=device)
    total = CHUNK_FRAMES * CHUNKS_PER_STREAM
    codes = torch.stack([
        torch.randint(0, config.codebook_size, (config.n_codebooks, total),
                      generator=torch.Generator().manual_seed(1 + s))
        for s in range(STREAMS)
    ])
    chunks = [codes[..., c * CHUNK_FRAMES:(c + 1) * CHUNK_FRAMES].contiguous().to(device)
              for c in range(CHUNKS_PER_STREAM)]
    pool = decoder.new_state_pool(num_slots=STREAMS)
    slot_index = torch.arange(STREAMS, device=device)

    def step(i: int) -> None:
        c = i % CHUNKS_PER_STREAM
        decoder.decode_slots(chunks[c], pool, slot_index, first_decode=c == 0)

    log(f"streaming: {STREAMS} streams x {CHUNK_FRAMES}-frame chunks, warmup {args.warmup}, "
        f"steps {args.steps}")
    elapsed = timed_steps(step, args.steps, args.warmup)
    audio_per_step = STREAMS * CHUNK_FRAMES / config.frame_rate
    value = args.steps * audio_per_step / elapsed
    log(f"streaming: {elapsed * 1e3 / args.steps:.3f} ms/step, {value:.1f} xRT")

    # instrumented pass: every launch between HIP events on the launch stream
    timer = LaunchTimer()
    decoder.timer = timer
    inst_steps = min(args.steps, CHUNKS_PER_STREAM)
    for i in range(inst_steps):
        step(args.warmup + args.steps + i)
    sync()
    decoder.timer = NO_TIMER
    summ = timer.summary()
    # the roofline kernel: the fused kernel with the largest share of the step (the residual
    # stack of the 96-channel stage: three residual units, conv k7 d 1/3/9 + Snake + conv k1 +
    # residual each, over 64 streams x 23 040 samples per launch; or a one-unit launch)
    fused = [k for k in summ if k.startswith(("stack", "unit"))]
    dom_kind = max(fused, key=lambda k: summ[k]["ms"])
    dom = summ[dom_kind]
    dom_flops_launch = dom["work"] / dom["launches"]
    dom_ms_launch = dom["ms"] / dom["launches"]
    achieved = dom_flops_launch / (dom_ms_launch * 1e-3) / 1e12
    mfma_kinds = [k for k in summ if k == "conv" or k.startswith(("unit", "stack"))]
    mfma_work = sum(summ[k]["work"] for k in mfma_kinds)
    mfma_ms = sum(summ[k]["ms"] for k in mfma_kinds)
    rvq = summ["rvq"]
    rvq_gbps = rvq["work"] / (rvq["ms"] * 1e-3) / 1e9
    # the decoder's MFMA convs: everything but the final one-channel conv
    final_macs = config.stage_channels()[-1] * config.kernel_size * config.hop_length
    expected = 2.0 * (dac_macs_per_frame(config) - final_macs) * STREAMS * CHUNK_FRAMES
    log(f"roofline kernel ({dom_kind}): {dom['launches'] / inst_steps:.0f} launches/step, "
        f"{dom_ms_launch * 1e3:.1f} us/launch, {achieved:.1f} TFLOP/s; all MFMA convs "
        f"{mfma_ms / inst_steps:.3f} ms/step, {mfma_work / (mfma_ms * 1e-3) / 1e12:.1f} TFLOP/s; "
        f"work/step {mfma_work / inst_steps / 1e12:.4f} TFLOP (layer list: {expected / 1e12:.4f})")
    for kind, v in sorted(summ.items()):
        log(f"  {kind:8s} {v['launches'] / inst_steps:5.1f} launches/step "
            f"{v['ms'] / inst_steps * 1e3:9.1f} us/step")
    kernel_ms = sum(v["ms"] for v in summ.values()) / inst_steps
    result = {
        "value": value,
        "ms_per_step": elapsed * 1e3 / args.steps,
        "config": {"workload": "streaming 24 kHz codec decode, 64 streams x 12-frame chunks, "
                               "36-frame context in per-layer slot state, 20 chunks per stream",
                   "streams": STREAMS, "chunk_frames": CHUNK_FRAMES,
                   "audio_s_per_step": audio_per_step, "codebooks": "16 x 2048 x 512",
                   "channels": 1536, "strides": [8, 8, 5, 6], "weights": "bf16"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": PMC_TRAFFIC_BYTES.get(dom_kind),
                     "traffic_source": PMC_TRAFFIC_SOURCE.get(dom_kind),
                     "kernel": KERNEL_NAMES.get(dom_kind, dom_kind),
                     "launches_per_step": dom["launches"] / inst_steps,
                     "flops_per_launch": dom_flops_launch, "mean_launch_ms": dom_ms_launch},
        "mfma_convs": {"TFLOPs": round(mfma_work / (mfma_ms * 1e-3) / 1e12, 1),
                       "ms_per_step": round(mfma_ms / inst_steps, 4)},
        "rvq_gather": {"in_step_GBps": round(rvq_gbps, 1),
                       "in_step_us": round(rvq["ms"] * 1e3 / rvq["launches"], 2)},
        "kernel_ms_per_step": round(kernel_ms, 4),
    }
    if not args.no_rvq_large:
        result["rvq_gather"]["large_batch"] = measure_rvq_large(device)
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(config, weights, frames=240, streams=10)
    return result


# HBM bytes per launch of the roofline kernel, from two rocprofv3 --pmc runs of
# `bench.py --only stack96` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by the
# same counter's reading for `bench.py --only copy` (a 1 GiB copy reads FETCH_SIZE = 512 MiB,
# WRITE_SIZE = 1024 MiB: fetch x 2, write x 1). Measured, not computed here: re-measure after a
# change to the kernel (profiles/residual_stack96_pmc.md holds the runs and their commands).
PMC_TRAFFIC_BYTES = {"stack96": round((146298.25 * 2 + 5894.0) * 1024)}
PMC_TRAFFIC_SOURCE = {"stack96": "profiles/residual_stack96_pmc.md: rocprofv3 FETCH_SIZE + "
                                 "WRITE_SIZE of `bench.py --only stack96`, copy-calibrated"}


def bench_hifigan(device) -> dict:
    """HiFiGAN mel -> wave, 16 clips of 500 mel frames (10 s each at 24 kHz), bf16."""
    from sglang_omni_amd.models import HifiGanVocoder, make_hifigan_weights
    from sglang_omni_amd.models.configs import HIFIGAN_24K, hifigan_macs_per_frame

    gen = torch.Generator().manual_seed(0)
    voc = HifiGanVocoder(make_hifigan_weights(HIFIGAN_24K, seed=0), HIFIGAN_24K, device=device)
    mel = (torch.randn(16, 80, 500, generator=gen) * 2 - 5).to(device)
    dt = timed_call(lambda: voc(mel))
    macs = hifigan_macs_per_frame(HIFIGAN_24K)
    return {"workload": "HiFiGAN mel->wave, 16 x 500 mel frames (160 s), bf16",
            "xRT": round(160.0 / dt, 1), "ms": round(dt * 1e3, 3),
            "TFLOPs": round(2.0 * macs * 16 * 500 / dt / 1e12, 1),
            "mfma_frac": round(2.0 * macs * 16 * 500 / dt / 1e12 / PEAK_BF16_TFLOPS, 4)}


def run_only(args, device) -> None:
    from sglang_omni_amd import _native as N
    from sglang_omni_amd.kernels.conv import FinalConv, residual_stack
    from sglang_omni_amd.models import DacCodecDecoder, make_dac_weights
    from sglang_omni_amd.models.configs import CODEC_24K

    if args.only == "copy":
        a = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device=device)
        b = torch.empty_like(a)
        fn = lambda: b.copy_(a)  # noqa: E731
        what = "1 GiB copy"
    else:
        decoder = DacCodecDecoder(make_dac_weights(CODEC_24K, seed=0), CODEC_24K, device=device)
        blk = decoder.blocks[-1]
        if blk.stack is None or blk.c_out != 96:
            raise SystemExit("the decoder's last block runs no 96-channel residual stack")
        gen = torch.Generator().manual_seed(0)
        x = (torch.randn(STREAMS, 23040, 96, generator=gen) * 0.3).to(device,
                                                                    decoder.residual_dtype)
        wave = torch.empty(STREAMS, 1, 23040, dtype=torch.float32, device=device)
        final = FinalConv(decoder.final_weight, decoder.final_bias, N.ACT_TANH, wave)
        last = blk.units[-1]
        fn = lambda: residual_stack(x, blk.stack, None, last.next_a, last.next_b,  # noqa: E731
                                    final=final, coef_table=blk.stack_coef)
        what = "residual stack + final conv, 96 channels, x [64, 23040, 96]"
    for _ in range(2):
        fn()
    sync()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.launches):
        fn()
    end.record()
    sync()
    log(f"{what}: {start.elapsed_time(end) * 1e3 / args.launches:.1f} us per launch "
        f"({args.launches} launches after 2 warmups)")


def graph_kernel_time(fn, launches: int) -> float:
    """Seconds per call of fn (a few short kernel launches), from one HIP-event pair around a
    HIP-graph replay of `launches` back-to-back calls: the GPU time of the kernels, not the
    host's per-call wrapper time, which exceeds a kernel of a few microseconds. The replay is
    checked against nothing here; the kernels' results are tested elsewhere."""
    fn()
    sync()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()  # warm the capture stream
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(launches):
                fn()
    torch.cuda.current_stream().wait_stream(stream)
    graph.replay()
    sync()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    graph.replay()
    end.record()
    sync()
    return start.elapsed_time(end) / 1e3 / launches


def timed_call(fn, reps: int = 3) -> float:
    fn()
    sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    sync()
    return (time.perf_counter() - t0) / reps


def bench_other_configs(device) -> dict:
    """xRT of the other decoder configurations (one call each, inputs resident in HBM)."""
    from sglang_omni_amd.models import DacCodecDecoder, make_dac_weights
    from sglang_omni_amd.models.configs import CODEC_24K, CODEC_24K_LONG, dac_macs_per_frame

    def mfma(frames: int, macs_per_frame: int, dt: float) -> dict:
        """The whole decoder's algorithmic FLOPs over its time, against the bf16 MFMA peak (the
        fp8-weight form multiplies in bf16 too)."""
        tflops = 2.0 * frames * macs_per_frame / dt / 1e12
        return {"TFLOPs": round(tflops, 1), "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4)}

    out = {}
    gen = torch.Generator().manual_seed(0)
    dec = DacCodecDecoder(make_dac_weights(CODEC_24K, seed=0), CODEC_24K, device=device)
    codes = torch.randint(0, 2048, (1, 16, 250), generator=gen).to(device)
    dt = timed_call(lambda: dec.from_indices(codes))
    out["single_utterance"] = {"workload": "24 kHz codec, 1 x 250 frames (20 s), bf16",
                               "xRT": round(20.0 / dt, 1), "ms": round(dt * 1e3, 3),
                               **mfma(250, dac_macs_per_frame(CODEC_24K), dt)}
    del dec
    out["hifigan"] = bench_hifigan(device)
    codes = torch.randint(0, 1024, (8, 32, 1500), generator=gen).to(device)
    long_weights = make_dac_weights(CODEC_24K_LONG, seed=0)
    for fmt in ("fp8", "bf16"):  # the same shape with each weight format
        dec = DacCodecDecoder(long_weights, CODEC_24K_LONG, device=device, weight_format=fmt)
        dt = timed_call(lambda: dec.from_indices(codes), reps=2)
        name = "fp8 e4m3" if fmt == "fp8" else "bf16"
        out[f"{fmt}_long_form"] = {"workload": f"24 kHz codec, {name} weights, 8 x 1500 frames "
                                               "(960 s), whole utterances",
                                   "xRT": round(960.0 / dt, 1), "ms": round(dt * 1e3, 3),
                                   **mfma(8 * 1500, dac_macs_per_frame(CODEC_24K_LONG), dt)}
        del dec
    return out


def bench_qwen3_code2wav(device, steps: int = 20, warmup: int = 3) -> dict:
    """The Qwen3-Omni code2wav (1024-hidden 8-layer pre-transformer, ConvNeXt upsamplers,
    1536-channel decoder, x1920 to 24 kHz; seeded random weights) in the streaming serving
    pattern: 64 streams, one step = one 12-frame chunk of every stream through the slot pool
    (K / V rings, conv histories), eagerly and replayed from a HIP graph; per-kind kernel times
    from HIP events on the launch stream."""
    from sglang_omni_amd.models import (CodecGraphRunner, GraphKey, Qwen3Code2WavDecoder,
                                        make_qwen3_code2wav_weights)
    from sglang_omni_amd.models.configs import QWEN3_CODE2WAV, qwen3_code2wav_macs_per_frame
    from sglang_omni_amd.utils.timing import NO_TIMER, LaunchTimer

    cfg = QWEN3_CODE2WAV
    dec = Qwen3Code2WavDecoder(make_qwen3_code2wav_weights(cfg, seed=0), cfg, device=device)
    codes = torch.stack([
        torch.randint(0, cfg.codebook_size, (cfg.num_quantizers, CHUNK_FRAMES * CHUNKS_PER_STREAM),
                      generator=torch.Generator().manual_seed(1 + s)) for s in range(STREAMS)])
    chunks = [codes[..., c * CHUNK_FRAMES:(c + 1) * CHUNK_FRAMES].contiguous().to(device)
              for c in range(CHUNKS_PER_STREAM)]
    pool = dec.new_state_pool(num_slots=STREAMS, capture_slots=STREAMS)
    index = torch.arange(STREAMS, device=device)
    audio_per_step = STREAMS * CHUNK_FRAMES * cfg.hop_length / cfg.sample_rate
    flops_per_step = 2.0 * qwen3_code2wav_macs_per_frame(cfg) * STREAMS * CHUNK_FRAMES

    def eager(i: int) -> None:
        c = i % CHUNKS_PER_STREAM
        dec.decode_slots(chunks[c], pool, index, first_decode=c == 0)

    out = {"workload": f"Qwen3-Omni code2wav, {STREAMS} streams x {CHUNK_FRAMES}-frame chunks "
                       f"(72-frame attention window and conv state in the slot pool), bf16",
           "gflop_per_step": round(flops_per_step / 1e9, 1)}
    dt = timed_steps(eager, steps, warmup) / steps
    out["eager"] = {"ms_per_step": round(dt * 1e3, 3), "xRT": round(audio_per_step / dt, 1)}
    runner = CodecGraphRunner(dec, pool, [GraphKey(STREAMS, CHUNK_FRAMES, "first"),
                                          GraphKey(STREAMS, CHUNK_FRAMES, "next")])
    runner.capture_all()

    def graphed(i: int) -> None:
        c = i % CHUNKS_PER_STREAM
        runner.run(chunks[c], index, first_decode=c == 0)

    dt = timed_steps(graphed, steps, warmup) / steps
    out["graph"] = {"ms_per_step": round(dt * 1e3, 3), "xRT": round(audio_per_step / dt, 1),
                    "TFLOPs": round(flops_per_step / dt / 1e12, 1)}
    timer = LaunchTimer()
    dec.timer = timer
    for i in range(CHUNKS_PER_STREAM):
        eager(i)
    sync()
    dec.timer = NO_TIMER
    kinds = {}
    for kind, v in timer.summary().items():
        entry = {"launches_per_step": round(v["launches"] / CHUNKS_PER_STREAM, 1),
                 "us_per_step": round(v["ms"] * 1e3 / CHUNKS_PER_STREAM, 1)}
        if v["work"]:
            entry["TFLOPs"] = round(v["work"] / (v["ms"] * 1e-3) / 1e12, 1)
        kinds[kind] = entry
    out["kernels"] = kinds
    return out


def bench_qwen3_tts(device, steps: int = 20, warmup: int = 3) -> dict:
    """The Qwen3-TTS tokenizer decoder (512-hidden 8-layer transformer with 16 x 64 attention,
    1024 latent, 1536-channel decoder, x1920; seeded random weights) through its incremental
    API: one state of 64 rows, each decode 12 fresh frames of every row."""
    from sglang_omni_amd.models import Qwen3TTSCodecDecoder, make_qwen3_code2wav_weights
    from sglang_omni_amd.models.configs import QWEN3_TTS_CODEC, qwen3_code2wav_macs_per_frame

    cfg = QWEN3_TTS_CODEC
    dec = Qwen3TTSCodecDecoder(make_qwen3_code2wav_weights(cfg, seed=0), cfg, device=device)
    codes = torch.randint(0, cfg.codebook_size,
                          (STREAMS, cfg.num_quantizers, CHUNK_FRAMES * CHUNKS_PER_STREAM),
                          generator=torch.Generator().manual_seed(1))
    chunks = [codes[..., c * CHUNK_FRAMES:(c + 1) * CHUNK_FRAMES].contiguous().to(device)
              for c in range(CHUNKS_PER_STREAM)]
    state = {"s": dec.init_state(STREAMS)}

    def step(i: int) -> None:
        c = i % CHUNKS_PER_STREAM
        if c == 0:
            state["s"] = dec.init_state(STREAMS)
        dec.decode(chunks[c], state["s"])

    dt = timed_steps(step, steps, warmup) / steps
    audio_per_step = STREAMS * CHUNK_FRAMES * cfg.hop_length / cfg.sample_rate
    flops = 2.0 * qwen3_code2wav_macs_per_frame(cfg) * STREAMS * CHUNK_FRAMES
    return {"workload": f"Qwen3-TTS tokenizer decoder, decode(codes, state) of {STREAMS} rows x "
                        f"{CHUNK_FRAMES} frames, bf16",
            "ms_per_step": round(dt * 1e3, 3), "xRT": round(audio_per_step / dt, 1),
            "TFLOPs": round(flops / dt / 1e12, 1)}


def bench_hift_transforms(device) -> dict:
    """HiFT's transforms at the HiFiGAN configuration's size (16 rows x 10 s at 24 kHz, n_fft 16,
    hop 4): the source spectrum (240 000 samples -> 18 x 60 001) and the fused iSTFT tail
    (18 x 60 001 channels-last -> 240 000 samples), as HBM bytes per second."""
    from sglang_omni_amd.kernels.hift import HiftStft

    st = HiftStft(torch.hann_window(16, periodic=True), 4, device=device)
    gen = torch.Generator().manual_seed(0)
    rows, samples = 16, 240000
    frames = samples // 4 + 1
    x = torch.randn(rows, samples, generator=gen).to(device)
    h = (torch.randn(rows, frames, 18, generator=gen) * 0.5 - 3.0).to(device)
    out = {}
    for name, fn, nbytes in (
            ("spectrum", lambda: st.spectrum(x), 4 * rows * (samples + 18 * frames)),
            ("istft_tail", lambda: st.tail(h), 4 * rows * (18 * frames + 4 * (frames - 1)))):
        dt = graph_kernel_time(fn, 20)
        gbps = nbytes / dt / 1e9
        out[name] = {"us": round(dt * 1e6, 1), "bytes": nbytes, "achieved_GBps": round(gbps, 1),
                     "frac": round(gbps / PEAK_HBM_GBPS, 4)}
    return out


def bench_egress(device) -> dict:
    """One streaming decode step's waveform (64 rows x 23 040 samples) leaving the device: the
    PCM16 egress kernel alone (HBM bytes per second), and the host-visible time of staging the
    step through the pinned ring and reading every row back (PCIe-inclusive), as float32 and as
    PCM16."""
    from sglang_omni_amd.kernels.egress import waveform_egress
    from sglang_omni_amd.scheduling import WaveformEgress

    rows, samples = 64, 23040
    w = (torch.rand(rows, 1, samples, device=device) * 2.2 - 1.1).contiguous()
    out = torch.empty(rows, samples, dtype=torch.int16, device=device)
    dt = graph_kernel_time(lambda: waveform_egress(w, format="pcm16", out=out), 50)
    nbytes = rows * samples * (4 + 2)
    line = {"pcm16_kernel": {"us": round(dt * 1e6, 2), "bytes": nbytes,
                             "achieved_GBps": round(nbytes / dt / 1e9, 1),
                             "frac": round(nbytes / dt / 1e9 / PEAK_HBM_GBPS, 4)}}
    ids = list(range(rows))
    for fmt in ("f32", "pcm16"):
        egress = WaveformEgress(device, format=fmt, depth=2)
        egress.stage_step(ids, w)
        egress.flush()
        reps = 20
        torch.cuda.synchronize(device)
        t0 = time.perf_counter()
        for _ in range(reps):
            egress.stage_step(ids, w)
            egress.flush()
        dt = (time.perf_counter() - t0) / reps
        host_bytes = rows * samples * (2 if fmt == "pcm16" else 4)
        line[f"step_to_host_{fmt}"] = {"ms": round(dt * 1e3, 3), "host_bytes": host_bytes,
                                       "GBps": round(host_bytes / dt / 1e9, 2)}
    return line


def bench_channel_embedding(device) -> dict:
    """MOSS-TTS's multi-channel input embedding: 33 channels (a 151 936-row text table and 32
    audio tables of 1 025 rows), hidden 2048, bf16, for a 64-row decode batch and a 4096-row
    prefill. Bytes are algorithmic: every gathered table row, the output rows and the int64 ids
    once (repeated audio rows may hit in cache)."""
    from sglang_omni_amd.kernels.channel_embedding import ChannelEmbeddingTables

    hidden, vocab = 2048, [151936] + [1025] * 32
    g = torch.Generator(device=device).manual_seed(0)
    weights = [torch.randn(v, hidden, device=device, dtype=torch.bfloat16, generator=g)
               for v in vocab]
    tables = ChannelEmbeddingTables()
    if not tables.refresh(weights):
        raise RuntimeError("the MOSS-TTS tables could not be fused")
    line = {}
    for rows, reps in ((64, 200), (4096, 50)):
        ids = torch.stack([torch.randint(0, v, (rows,), device=device, generator=g)
                           for v in vocab], dim=1)
        dt = graph_kernel_time(lambda: tables.embed(ids, weights), reps)
        nbytes = rows * (len(vocab) * hidden * 2 + hidden * 2 + len(vocab) * 8)
        line[f"rows_{rows}"] = {"us": round(dt * 1e6, 2), "bytes": nbytes,
                                "achieved_GBps": round(nbytes / dt / 1e9, 1),
                                "frac": round(nbytes / dt / 1e9 / PEAK_HBM_GBPS, 4)}
    return line


def calibrate(device) -> dict:
    """The box's practical peaks: a 1 GiB device copy (HBM) and a 8192^3 bf16 GEMM (torch's
    hipBLASLt, the MFMA reference point)."""
    a = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device=device)
    b = torch.empty_like(a)
    dt = timed_call(lambda: b.copy_(a), reps=5)
    copy = 2.0 * a.numel() * 4 / dt / 1e9
    del a, b
    x = torch.randn(8192, 8192, device=device).to(torch.bfloat16)
    y = torch.randn(8192, 8192, device=device).to(torch.bfloat16)
    dt = timed_call(lambda: torch.matmul(x, y), reps=5)
    return {"copy_GBps": round(copy, 1), "bf16_gemm_8192_TFLOPs": round(2.0 * 8192 ** 3 / dt / 1e12, 1)}


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=40)
    # the GPU's clocks ramp over the first ~10 decode steps (the stack launch runs 1.42 ms in the
    # first, 1.13 ms from the tenth on): the warm-up covers the ramp
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--workload", default="streaming64")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-rvq-large", action="store_true")
    parser.add_argument("--only", choices=["stack96", "copy", "qwen3_code2wav", "hifigan"],
                        help="run one kernel alone (hardware-counter profiles; prints no JSON), "
                             "or only the Qwen3-Omni code2wav or HiFiGAN leg (prints its JSON)")
    parser.add_argument("--launches", type=int, default=2)
    parser.add_argument("--no-other-configs", action="store_true",
                        help="skip the xRT of the other configurations and the peak calibration")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this library has no multi-GPU path (asked for "
              f"--gpus {args.gpus}); streams shard across GPUs by process (one decoder, "
              "slot pool and stream set per GPU, no collective on the decode path).",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    device = torch.device("cuda", 0)
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.only == "qwen3_code2wav":
        print(json.dumps(bench_qwen3_code2wav(device)), flush=True)
        return
    if args.only == "hifigan":
        print(json.dumps(bench_hifigan(device)), flush=True)
        return
    if args.only:
        run_only(args, device)
        return
    if args.workload != "streaming64":
        raise SystemExit(f"unknown workload {args.workload}")
    r = bench_streaming(args, device)
    line = {
        "metric": METRIC,
        "value": round(r["value"], 2),
        "unit": "audio-s/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform random codes, seeded random-init weights)",
        "config": r["config"],
        "roofline": r["roofline"],
        "mfma_convs": r["mfma_convs"],
        "rvq_gather": r["rvq_gather"],
        "kernel_ms_per_step": r["kernel_ms_per_step"],
    }
    if "cpu_baseline" in r:
        line["cpu_baseline"] = r["cpu_baseline"]
    if not args.no_other_configs:
        log("other configurations ...")
        line["other_configs"] = bench_other_configs(device)
        line["hift_transforms"] = bench_hift_transforms(device)
        line["egress"] = bench_egress(device)
        line["channel_embedding"] = bench_channel_embedding(device)
        line["qwen3_code2wav"] = bench_qwen3_code2wav(device)
        line["qwen3_tts_codec"] = bench_qwen3_tts(device)
        line["calibration"] = calibrate(device)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
