"""Decode benchmark: the KV-cached Whisper decoder token loop on one MI355X.

Workload (default): the small shape — d_model 768, 12 heads, 12 layers, vocab
51865, fp16-stored weights (fp32 accumulate), encoder states 1500 x 768 N(0,1),
batch 1 — decoding from a 4-token start-of-transcript prefix, cross K/V
projected once per sequence. A "step" is one single-token decoder step plus its
greedy argmax, the token fed back on the device (Decoder::step followed by
Argmax::encode, as Whisper::encodeStep records them). The timed region is
exactly --steps such steps, bracketed by synchronisation, inputs resident in
HBM; warm-up steps run in a sequence of their own first. With the default 224
steps the self-attention KV grows 5..228 keys over the timed steps.

The JSON line reports decode tokens/s, ms/step, the HBM roofline of the step
(algorithmic bytes per step / measured step time against 8 TB/s) and the CPU
oracle timed on the host cores over a bounded sample of the same workload,
whose tokens are also checked against the GPU's.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def step_bytes(shape, weight_bytes: int, position: int, streams: int = 1) -> int:
    """Algorithmic HBM bytes of one single-token step at `position` (keys
    attended = position + 1): every projection and the tied logits weight once,
    the fp32 biases and norms, the cross K/V, the self K/V so far, the embedding
    rows, the new K/V rows and the logits row."""
    d, L, f, V, T = shape.width, shape.layers, shape.feed_forward_width, shape.vocabulary_size, shape.cross_positions
    weights = L * (4 * d * d + 2 * d * d + 2 * d * f) * weight_bytes + V * d * weight_bytes
    params = (L * (12 * d + f) + 2 * d) * 4
    n = position + 1
    per_stream = 2 * L * T * d * 4 + 2 * L * n * d * 4 + 2 * d * 4 + 2 * L * d * 4 + V * 4
    return weights + params + streams * per_stream


def measured_traffic(workload: str, unfused: bool):
    """HBM bytes per step-kernel launch as the FETCH_SIZE and WRITE_SIZE
    counters measured them (each scaled by its reading for a plain copy of
    known size), from the summary committed under profiles/; None when there
    is no summary for this workload and path."""
    if unfused:
        return None
    path = os.path.join(ROOT, "profiles", f"step_kernel_{workload}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def cpu_baseline(shape, decoder_file, encoder, prompt, gpu_tokens, budget_s: float):
    """The oracle (the C restatement of the reference's double-precision
    decoder) on the host cores over a bounded sample: the prompt step, then
    single-token steps until the time budget is spent."""
    import numpy as np
    from oracle import load_oracle
    from whispereacp_amd import synthetic as S

    oracle = load_oracle()
    cores = min(16, os.cpu_count() or 1)
    oracle.set_threads(cores)
    tensors = [decoder_file[n].floats() for n in S.canonical_names(shape.layers)]
    session = oracle.session(shape, tensors)
    t0 = time.perf_counter()
    session.begin(encoder)
    begin_s = time.perf_counter() - t0
    _, logits = session.step(prompt)
    tokens = [int(np.argmax(logits[-1]))]
    steps, spent = 0, 0.0
    while spent < budget_s and steps < len(gpu_tokens) - 1:
        t = time.perf_counter()
        _, logits = session.step([tokens[-1]])
        spent += time.perf_counter() - t
        tokens.append(int(np.argmax(logits[0])))
        steps += 1
    per_step = spent / max(steps, 1)
    match = tokens == gpu_tokens[:len(tokens)]
    return {
        "value": round(1.0 / per_step, 3),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{steps} single-token steps after the 4-token prompt (positions 4..{3 + steps}) of the same "
                   f"workload in double precision; begin_sequence (cross K/V over 1500 rows) took "
                   f"{begin_s:.1f} s and is excluded"),
        "ms_per_step": round(per_step * 1e3, 2),
    }, {"steps_checked": len(tokens), "tokens_match": bool(match)}


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=None, help="timed steps (default: the workload's own)")
    parser.add_argument("--warmup", type=int, default=16)
    parser.add_argument("--workload", default="small", choices=["base.en", "small", "medium", "large-v3"])
    parser.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of oracle time (0: skip)")
    parser.add_argument("--unfused", action="store_true", help="time the per-op kernel sequence instead")
    parser.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                        help="only run a plain device-to-device copy of BYTES (the reference reading for the "
                             "FETCH_SIZE/WRITE_SIZE counters) and exit")
    args = parser.parse_args()

    if args.copy_calibration > 0:
        import torch
        src = torch.ones(args.copy_calibration, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": args.copy_calibration, "copies": 4}))
        return

    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from whispereacp_amd import synthetic as S
    from whispereacp_amd.decoder import Decoder, to_device

    w = S.WORKLOADS[args.workload]
    if args.steps is None:
        args.steps = w["steps"]
    if w["streams"] > 1:
        bench_streams(args, w)
        return
    shape = S.workload_shape(args.workload)
    prompt = S.SOT_PREFIX[shape.vocabulary_size]
    if len(prompt) + args.steps > shape.max_positions or len(prompt) + args.warmup > shape.max_positions:
        print(f"--steps and --warmup each fit {shape.max_positions - len(prompt)} steps in one sequence",
              file=sys.stderr)
        sys.exit(2)
    dtype = w["dtype"]
    weight_bytes = 4 if dtype == "F32" else 2

    print(f"[bench] generating {args.workload} weights ({dtype})", file=sys.stderr, flush=True)
    decoder_file = S.workload_decoder_file(shape, dtype, 1000)
    encoder = S.normal_encoder_output(shape.cross_positions, shape.width, 7)
    torch.cuda.set_device(0)
    decoder = Decoder(shape, decoder_file, packing="ExactHalf")
    decoder.set_fused(not args.unfused)
    enc = to_device(encoder)
    V = shape.vocabulary_size
    slots = torch.zeros(shape.max_positions + 1, dtype=torch.int32, device="cuda")
    prompt_logits = torch.empty((len(prompt), V), dtype=torch.float32, device="cuda")
    step_logits = torch.empty((1, V), dtype=torch.float32, device="cuda")

    def open_sequence():
        slots[:len(prompt)] = torch.tensor(prompt, dtype=torch.int32, device="cuda")
        decoder.begin_sequence(enc)
        decoder.step(slots[:len(prompt)], len(prompt), prompt_logits)
        decoder.argmax(prompt_logits[-1:], 1, V, None, slots[len(prompt):len(prompt) + 1])

    def run_steps(count):
        base = len(prompt)
        for j in range(1, count + 1):
            decoder.step_and_sample(slots[base + j - 1:base + j], step_logits, None, slots[base + j:base + j + 1])

    print("[bench] warm-up", file=sys.stderr, flush=True)
    open_sequence()
    run_steps(args.warmup)
    torch.cuda.synchronize()

    print("[bench] timed region", file=sys.stderr, flush=True)
    open_sequence()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    host0 = time.perf_counter()
    start.record()
    run_steps(args.steps)
    stop.record()
    enqueue_s = time.perf_counter() - host0
    torch.cuda.synchronize()
    host_s = time.perf_counter() - host0
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = gpu_ms / args.steps
    gpu_tokens = slots[len(prompt):len(prompt) + args.steps + 1].cpu().numpy().tolist()

    positions = range(len(prompt), len(prompt) + args.steps)
    bytes_total = sum(step_bytes(shape, weight_bytes, p) for p in positions)
    bytes_per_step = bytes_total / args.steps
    achieved = bytes_per_step / (ms_per_step * 1e-3) / 1e9

    traffic = measured_traffic(args.workload, args.unfused)

    baseline, parity = None, None
    if args.cpu_budget > 0:
        print("[bench] cpu baseline (oracle)", file=sys.stderr, flush=True)
        baseline, parity = cpu_baseline(shape, decoder_file, encoder, prompt, gpu_tokens, args.cpu_budget)

    line = {
        "metric": "decode tokens/s and ms/step at batch 1, % of HBM roofline (d=768 shapes)",
        "value": round(args.steps / (gpu_ms * 1e-3), 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16-weights/f32" if dtype == "F16" else "f32",
        "data": "synthetic: N(0,0.02) weights (LayerNorm gamma 1, beta 0), N(0,1) encoder states, fixed seeds",
        "config": {"workload": f"{args.workload} decoder: d_model {shape.width}, {shape.heads} heads, "
                               f"{shape.layers} layers, vocab {V}, {dtype} weights, 1500 cross positions, "
                               f"batch 1, {args.steps} single-token greedy steps after a 4-token prefix",
                   "path": "per-op kernel sequence" if args.unfused else "fused single-token step",
                   "global_batch": 1, "seq_len": len(prompt) + args.steps, "parallelism": "none (one GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "step_kernel (one persistent launch per decode step)" if not args.unfused
                     else "per-op kernel sequence",
                     "bytes_per_step": round(bytes_per_step)},
        "cpu_baseline": baseline,
        "parity": parity,
        "host_seconds": round(host_s, 4),
        "host_enqueue_seconds": round(enqueue_s, 4),
    }
    print(json.dumps(line))


def bench_streams(args, w):
    """The batched configurations: w["streams"] independent sequences, each
    with its own N(0,1) encoder states, decoded together (BatchedDecoder), one
    token per stream per step. With large-v3 the cross K/V projection of every
    stream runs inside the timed region, as that configuration is quoted."""
    import numpy as np
    import torch
    from whispereacp_amd import synthetic as S
    from whispereacp_amd.decoder import BatchedDecoder, to_device

    shape = S.workload_shape(args.workload)
    streams, dtype = w["streams"], w["dtype"]
    prompt = S.SOT_PREFIX[shape.vocabulary_size]
    if len(prompt) + args.steps > shape.max_positions or len(prompt) + args.warmup > shape.max_positions:
        print(f"--steps and --warmup each fit {shape.max_positions - len(prompt)} steps in one sequence",
              file=sys.stderr)
        sys.exit(2)
    begin_timed = args.workload == "large-v3"
    print(f"[bench] generating {args.workload} weights ({dtype}) and {streams} encoder outputs", file=sys.stderr,
          flush=True)
    decoder_file = S.workload_decoder_file(shape, dtype, 1000)
    encoders = [S.normal_encoder_output(shape.cross_positions, shape.width, 7 + s) for s in range(streams)]
    torch.cuda.set_device(0)
    decoder = BatchedDecoder(shape, decoder_file, streams=streams)
    enc = to_device(np.ascontiguousarray(np.stack(encoders)))
    V = shape.vocabulary_size
    t = len(prompt)
    prompt_tokens = torch.tensor([prompt] * streams, dtype=torch.int32, device="cuda")
    # Token ring [position][stream]: the prompt step's argmax lands in row t,
    # each replayed step reads row p and writes row p + 1.
    ring = torch.zeros((shape.max_positions + 1, streams), dtype=torch.int32, device="cuda")
    ring[:t] = torch.tensor(prompt, dtype=torch.int32, device="cuda")[:, None].expand(t, streams)
    prompt_logits = torch.empty((streams * t, V), dtype=torch.float32, device="cuda")
    step_logits = torch.empty((streams, V), dtype=torch.float32, device="cuda")

    def open_sequence():
        decoder.begin(enc)
        decoder.step(prompt_tokens, t, prompt_logits, None, ring[t])

    def run_steps(count):
        for _ in range(count):
            decoder.ring_step(ring, step_logits, None)

    print("[bench] warm-up", file=sys.stderr, flush=True)
    open_sequence()
    run_steps(args.warmup)
    torch.cuda.synchronize()

    print("[bench] timed region", file=sys.stderr, flush=True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if begin_timed:
        torch.cuda.synchronize()
        host0 = time.perf_counter()
        start.record()
        open_sequence()
    else:
        open_sequence()
        torch.cuda.synchronize()
        host0 = time.perf_counter()
        start.record()
    run_steps(args.steps)
    stop.record()
    enqueue_s = time.perf_counter() - host0
    torch.cuda.synchronize()
    host_s = time.perf_counter() - host0
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = gpu_ms / args.steps
    tokens = ring[t:t + args.steps + 1].cpu().numpy().T

    weight_bytes = 4 if dtype == "F32" else 2
    positions = range(t, t + args.steps)
    bytes_per_step = sum(step_bytes(shape, weight_bytes, p, streams) for p in positions) / args.steps
    achieved = bytes_per_step / (ms_per_step * 1e-3) / 1e9

    baseline, parity = None, None
    if args.cpu_budget > 0:
        print("[bench] cpu baseline (oracle, stream 0)", file=sys.stderr, flush=True)
        baseline, parity = cpu_baseline(shape, decoder_file, encoders[0], prompt, tokens[0].tolist(),
                                        args.cpu_budget)
        baseline["sample"] = "one stream: " + baseline["sample"]

    line = {
        "metric": f"decode tokens/s and ms/step, {streams} independent streams",
        "value": round(streams * args.steps / (gpu_ms * 1e-3), 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("f16" if dtype == "F16" else "bf16") + "-weights/f32",
        "data": "synthetic: N(0,0.02) weights (LayerNorm gamma 1, beta 0), N(0,1) encoder states per stream",
        "config": {"workload": f"{args.workload} decoder: d_model {shape.width}, {shape.heads} heads, "
                               f"{shape.layers} layers, vocab {V}, {dtype} weights, 1500 cross positions, "
                               f"{streams} streams, {args.steps} single-token greedy steps after a 4-token prefix"
                               + (", cross K/V projection of every stream timed" if begin_timed else ""),
                   "path": "batched per-op kernels (matrix-core products), one HIP graph replay per step",
                   "global_batch": streams, "seq_len": t + args.steps, "parallelism": "none (one GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole step (batched per-op kernels)", "bytes_per_step": round(bytes_per_step)},
        "cpu_baseline": baseline,
        "parity": parity,
        "host_seconds": round(host_s, 4),
        "host_enqueue_seconds": round(enqueue_s, 4),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
