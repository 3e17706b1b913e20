"""Decode benchmark: the KV-cached Whisper decoder token loop on one MI355X.

Workload (default): the small shape — d_model 768, 12 heads, 12 layers, vocab
51865, fp16-stored weights (fp32 accumulate), encoder states 1500 x 768 N(0,1),
batch 1 — decoding 224 single-token greedy steps after a 4-token
start-of-transcript prefix, cross K/V projected once per sequence. A "step" is
one single-token decoder step plus its greedy argmax, the token fed back on the
device (Decoder::step followed by Argmax::encode, as Whisper::encodeStep
records them). Inputs are resident in HBM; warm-up steps run in a sequence of
their own first.

Timing follows the reference's benchmark protocol (Benchmark/README.md:62-106):
one warm-up, then --runs timed runs (10 by default) of the whole sequence, and
the median run is reported with the fastest and slowest beside it. Within a
run, with --steps equal to the workload's own step count (the default) the
whole sequence is one event-bracketed region, the self-attention KV growing
5..228 keys. With fewer, the whole sequence still runs, and --steps consecutive
steps from its middle are bracketed by one pair of HIP events on the decoder's
stream (nothing synchronises inside the sequence, so the launch queue never
drains); the bytes per step are averaged over the same positions. Every run
must decode the same tokens.

The JSON line reports decode tokens/s, ms/step, the HBM roofline of the step
(algorithmic bytes per step / measured step time against 8 TB/s) and the CPU
oracle timed on the host cores over a bounded sample of the same workload —
on one thread (the reference oracle's own model) and on every usable core —
whose tokens are also checked against the GPU's. `--workload tiny.en
--cpu-only` runs only the oracle at the tiny.en shape, the configuration the
reference runs on the CPU.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# MI355X dense matrix-core peaks (TFLOP/s) by the products' weight storage.
MFMA_PEAK_TFLOPS = {"F16": 2500.0, "BF16": 2500.0, "F32": 157.3}
# The encoder legs' projection storage per model (large-v3 ships bf16).
ENCODER_DTYPES = {"tiny.en": "F16", "base.en": "F16", "small": "F16", "medium": "F16", "large-v3": "BF16"}
# Published: tiny.en decoding jfk.wav, 25 steps, median of 30 runs, Apple M5 Max (README.md:44-53).
REFERENCE_TINY_DECODE_S = 0.0123
METRIC = "decode tokens/s and ms/step at batch 1, % of HBM roofline (d=768 shapes)"


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
    known size), and the positions they were measured over, from the summary
    committed under profiles/; (None, None) when there is none."""
    if unfused:
        return None, None
    path = os.path.join(ROOT, "profiles", f"step_kernel_{workload}_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        data = json.load(f)
    return data.get("bytes_per_launch"), data.get("positions")


def host_description():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"nproc": os.cpu_count(), "usable_cpus": usable, "cpu_model": model}


def all_cores(host) -> int:
    """Every CPU this process may run on, within the OMP_NUM_THREADS share
    when the environment sets one."""
    cores = host["usable_cpus"]
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        cores = min(cores, int(env))
    return max(1, cores)


def cpu_baseline(shape, decoder_file, encoder, prompt, gpu_tokens, budget_s: float):
    """The oracle (the C restatement of the reference's double-precision
    decoder, KV-cached) on the host: begin_sequence and the prompt step on every
    usable core, then single-token steps on every core for half the budget and
    on one thread for the other half, continuing the same sequence (the
    oracle's threaded loops keep each output's summation order, so the threads
    change nothing in the results). begin_sequence on one thread is timed over
    a tenth of the encoder rows and scaled (its cost is linear in the rows).
    The tokens are compared with the GPU's."""
    import numpy as np
    from oracle import load_oracle
    from whispereacp_amd import synthetic as S

    host = host_description()
    cores = all_cores(host)
    oracle = load_oracle()
    tensors = [decoder_file[n].floats() for n in S.canonical_names(shape.layers)]

    oracle.set_threads(1)
    sub_rows = max(1, shape.cross_positions // 10)
    probe = oracle.session(shape, tensors)
    t0 = time.perf_counter()
    probe.begin(encoder, sub_rows)
    begin_single_s = (time.perf_counter() - t0) * shape.cross_positions / sub_rows
    del probe

    oracle.set_threads(cores)
    session = oracle.session(shape, tensors)
    t0 = time.perf_counter()
    session.begin(encoder)
    begin_s = time.perf_counter() - t0
    _, logits = session.step(prompt)
    tokens = [int(np.argmax(logits[-1]))]
    limit = len(gpu_tokens) - 1

    def run(threads, budget, most):
        oracle.set_threads(threads)
        steps, spent = 0, 0.0
        first = session.position
        while spent < budget and steps < most and len(tokens) - 1 < limit:
            t = time.perf_counter()
            _, step_logits = session.step([tokens[-1]])
            spent += time.perf_counter() - t
            tokens.append(int(np.argmax(step_logits[0])))
            steps += 1
        return steps, spent, first

    # The threaded sample leaves at least half the sequence to the single-thread one.
    many_steps, many_s, many_first = run(cores, budget_s / 2, max(1, limit // 2))
    one_steps, one_s, one_first = run(1, budget_s / 2, limit)
    oracle.set_threads(cores)
    many_per = many_s / max(many_steps, 1)
    one_per = one_s / max(one_steps, 1)
    match = tokens == gpu_tokens[:len(tokens)]
    return {
        "value": round(1.0 / many_per, 3),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{many_steps} single-token steps (positions {many_first}..{many_first + many_steps - 1}) on "
                   f"{cores} threads, then {one_steps} (positions {one_first}..{one_first + one_steps - 1}) on one "
                   f"thread, of the same workload's sequence in double precision; begin_sequence (cross K/V over "
                   f"{shape.cross_positions} rows) timed apart"),
        "ms_per_step": round(many_per * 1e3, 2),
        "begin_sequence_s": round(begin_s, 3),
        "single_thread": {"value": round(1.0 / one_per, 3), "unit": "tokens/s", "cores": 1,
                          "ms_per_step": round(one_per * 1e3, 2),
                          "begin_sequence_s": round(begin_single_s, 3),
                          "begin_sequence_note": f"timed over {sub_rows} of {shape.cross_positions} rows, scaled"},
        "host": host,
    }, {"steps_checked": len(tokens), "tokens_match": bool(match)}


def cpu_only(args, w):
    """The reference's CPU configuration: the oracle alone, on one thread, over
    the workload's whole sequence (begin_sequence, the prompt step and every
    single-token step), the median of --repeats runs after one warm-up run, as
    the reference's benchmark takes it."""
    import numpy as np
    from oracle import load_oracle
    from whispereacp_amd import synthetic as S

    shape = S.workload_shape(args.workload)
    prompt = S.SOT_PREFIX[shape.vocabulary_size]
    steps = args.steps
    print(f"[bench] generating {args.workload} weights ({w['dtype']})", file=sys.stderr, flush=True)
    decoder_file = S.workload_decoder_file(shape, w["dtype"], w["seed"])
    encoder = S.normal_encoder_output(shape.cross_positions, shape.width, 7)
    host = host_description()
    oracle = load_oracle()
    oracle.set_threads(1)
    tensors = [decoder_file[n].floats() for n in S.canonical_names(shape.layers)]
    runs = []
    tokens = None
    for r in range(args.repeats + 1):
        print(f"[bench] oracle run {r} ({'warm-up' if r == 0 else 'timed'})", file=sys.stderr, flush=True)
        session = oracle.session(shape, tensors)
        t0 = time.perf_counter()
        session.begin(encoder)
        t1 = time.perf_counter()
        _, logits = session.step(prompt)
        seq = [int(np.argmax(logits[-1]))]
        t2 = time.perf_counter()
        for _ in range(steps):
            _, logits = session.step([seq[-1]])
            seq.append(int(np.argmax(logits[0])))
        t3 = time.perf_counter()
        if tokens is not None:
            assert seq == tokens, "the oracle's tokens differ between runs"
        tokens = seq
        if r > 0:
            runs.append((t1 - t0, t2 - t1, t3 - t2))
    runs.sort(key=lambda x: x[2])
    begin_s, prompt_s, steps_s = runs[len(runs) // 2]
    per = steps_s / steps
    print(json.dumps({
        "metric": METRIC,
        "value": round(1.0 / per, 3),
        "unit": "tokens/s",
        "n_gpus": 0,
        "steps": steps,
        "warmup": 1,
        "ms_per_step": round(per * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic: N(0,0.02) weights (LayerNorm gamma 1, beta 0), N(0,1) encoder states, fixed seeds",
        "config": {"workload": f"{args.workload} decoder on the CPU oracle (one thread, double precision): d_model "
                               f"{shape.width}, {shape.heads} heads, {shape.layers} layers, vocab "
                               f"{shape.vocabulary_size}, {w['dtype']} weights, 1500 cross positions, batch 1, "
                               f"{steps} single-token greedy steps after a 4-token prefix",
                   "path": "oracle (CPU)", "global_batch": 1, "seq_len": len(prompt) + steps,
                   "parallelism": "none (one thread)"},
        "begin_sequence_s": round(begin_s, 3),
        "prompt_step_s": round(prompt_s, 4),
        "decode_s": round(steps_s, 4),
        "repeats": args.repeats,
        "tokens": tokens,
        "host": host,
    }))


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=None, help="timed steps (default: the workload's own)")
    parser.add_argument("--warmup", type=int, default=16)
    parser.add_argument("--runs", type=int, default=10,
                        help="timed runs of the whole sequence; the median is reported (decoder workloads)")
    parser.add_argument("--workload", default="small",
                        choices=["tiny.en", "base.en", "small", "medium", "large-v3"]
                        + ["encoder-" + n for n in ENCODER_DTYPES] + ["transcribe-tiny.en"])
    parser.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of oracle time (0: skip)")
    parser.add_argument("--cpu-only", action="store_true",
                        help="run only the oracle on one thread (the reference's CPU configuration)")
    parser.add_argument("--repeats", type=int, default=5, help="timed oracle runs with --cpu-only")
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

    from whispereacp_amd import synthetic as S

    if args.workload.startswith("encoder-"):
        bench_encoder(args)
        return
    if args.workload == "transcribe-tiny.en":
        bench_transcribe(args)
        return
    w = S.WORKLOADS[args.workload]
    if args.steps is None:
        args.steps = w["steps"]
    if args.steps <= 0 or args.warmup < 0 or args.runs <= 0:
        print("--steps and --runs must be positive and --warmup not negative", file=sys.stderr)
        sys.exit(2)
    if args.cpu_only:
        cpu_only(args, w)
        return
    if w["streams"] > 1:
        bench_streams(args, w)
        return
    bench_single(args, w)


def check_watchdog(decoder, where: str):
    status = decoder.device_status()
    if status != 0:
        decoder.device_status(clear=True)
        print(f"[bench] the persistent step's watchdog tripped during the {where}: its steps ended early and the "
              f"run is not a measurement", file=sys.stderr)
        sys.exit(3)


def bench_single(args, w):
    import numpy as np
    import torch
    from whispereacp_amd import synthetic as S
    from whispereacp_amd.decoder import Decoder, to_device

    shape = S.workload_shape(args.workload)
    prompt = S.SOT_PREFIX[shape.vocabulary_size]
    total = max(args.steps, w["steps"])
    if len(prompt) + total > shape.max_positions or len(prompt) + args.warmup > shape.max_positions:
        print(f"--steps and --warmup each fit {shape.max_positions - len(prompt)} steps in one sequence",
              file=sys.stderr)
        sys.exit(2)
    dtype = w["dtype"]
    weight_bytes = 4 if dtype == "F32" else 2

    print(f"[bench] generating {args.workload} weights ({dtype})", file=sys.stderr, flush=True)
    decoder_file = S.workload_decoder_file(shape, dtype, w["seed"])
    encoder = S.normal_encoder_output(shape.cross_positions, shape.width, 7)
    torch.cuda.set_device(0)
    decoder = Decoder(shape, decoder_file, packing="ExactHalf")
    decoder.set_fused(not args.unfused)
    enc = to_device(encoder)
    V = shape.vocabulary_size
    slots = torch.zeros(shape.max_positions + 1, dtype=torch.int32, device="cuda")
    prompt_logits = torch.empty((len(prompt), V), dtype=torch.float32, device="cuda")
    step_logits = torch.empty((1, V), dtype=torch.float32, device="cuda")
    base = len(prompt)

    def open_sequence():
        """begin_sequence and the prefix in one step; returns the event pair
        around the prefix step."""
        slots[:base] = torch.tensor(prompt, dtype=torch.int32, device="cuda")
        decoder.begin_sequence(enc)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        decoder.step(slots[:base], base, prompt_logits)
        stop.record()
        decoder.argmax(prompt_logits[-1:], 1, V, None, slots[base:base + 1])
        return start, stop

    def one_step(j):
        # step j (1-based) reads the token at position base + j - 1
        decoder.step_and_sample(slots[base + j - 1:base + j], step_logits, None, slots[base + j:base + j + 1])

    print("[bench] warm-up", file=sys.stderr, flush=True)
    open_sequence()
    for j in range(1, args.warmup + 1):
        one_step(j)
    torch.cuda.synchronize()
    check_watchdog(decoder, "warm-up")

    contiguous = args.steps == total
    # The timed steps: the whole sequence, or --steps consecutive steps from
    # its middle, one event pair around them (an event pair around each of a
    # few scattered steps would add the events' own cost to every step).
    first_timed = (total - args.steps) // 2
    timed = list(range(first_timed, first_timed + args.steps))

    def timed_run():
        """One whole sequence; returns (ms per timed step, tokens, host s,
        enqueue s, prefix step ms)."""
        prefix = open_sequence()
        torch.cuda.synchronize()
        prefix_ms = prefix[0].elapsed_time(prefix[1])
        host0 = time.perf_counter()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for j in range(1, total + 1):
            if j - 1 == timed[0]:
                start.record()
            one_step(j)
            if j - 1 == timed[-1]:
                stop.record()
        enqueue = time.perf_counter() - host0
        torch.cuda.synchronize()
        host = time.perf_counter() - host0
        check_watchdog(decoder, "timed region")
        gpu_ms = start.elapsed_time(stop)
        return gpu_ms / args.steps, slots[base:base + total + 1].cpu().numpy().tolist(), host, enqueue, prefix_ms

    print(f"[bench] timed region: {args.runs} runs", file=sys.stderr, flush=True)
    runs = [timed_run() for _ in range(args.runs)]
    run_ms = [r[0] for r in runs]
    ms_per_step = statistics.median(run_ms)
    gpu_tokens = runs[0][1]
    if any(r[1] != gpu_tokens for r in runs):
        print("[bench] the timed runs decoded different tokens", file=sys.stderr)
        sys.exit(3)
    median_run = min(runs, key=lambda r: abs(r[0] - ms_per_step))
    host_s, enqueue_s = median_run[2], median_run[3]

    positions = [base + j for j in timed]
    bytes_per_step = sum(step_bytes(shape, weight_bytes, p) for p in positions) / len(positions)
    achieved = bytes_per_step / (ms_per_step * 1e-3) / 1e9

    traffic, traffic_positions = measured_traffic(args.workload, args.unfused)

    baseline, parity = None, None
    if args.cpu_budget > 0:
        print("[bench] cpu baseline (oracle)", file=sys.stderr, flush=True)
        baseline, parity = cpu_baseline(shape, decoder_file, encoder, prompt, gpu_tokens, args.cpu_budget)

    sampling = ("every step" if contiguous else
                f"{args.steps} consecutive steps from the middle of the {total}, one HIP event pair around them")
    line = {
        "metric": METRIC,
        "value": round(1e3 / ms_per_step, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"F16": "f16-weights/f32", "BF16": "bf16-weights/f32"}.get(dtype, "f32"),
        "data": "synthetic: N(0,0.02) weights (LayerNorm gamma 1, beta 0), N(0,1) encoder states, fixed seeds",
        "config": {"workload": f"{args.workload} decoder: d_model {shape.width}, {shape.heads} heads, "
                               f"{shape.layers} layers, vocab {V}, {dtype} weights, 1500 cross positions, "
                               f"batch 1, {total} single-token greedy steps after a 4-token prefix "
                               f"(timed: {sampling})",
                   "path": "per-op kernel sequence" if args.unfused else "fused single-token step",
                   "global_batch": 1, "seq_len": base + total, "parallelism": "none (one GPU)",
                   "timed_positions": f"{positions[0]}..{positions[-1]}"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_positions": traffic_positions,
                     "kernel": "step_kernel (one persistent launch per decode step)" if not args.unfused
                     else "per-op kernel sequence",
                     "bytes_per_step": round(bytes_per_step)},
        "cpu_baseline": baseline,
        "parity": parity,
        "prefix_step": {"tokens": base, "ms": round(statistics.median(r[4] for r in runs), 4),
                        "note": "the 4-token prefix as one decoder step (one multi-token launch), median of the runs"},
        "runs": run_summary(run_ms),
        "host_seconds": round(host_s, 4),
        "host_enqueue_seconds": round(enqueue_s, 4),
    }
    print(json.dumps(line))


def run_summary(run_ms):
    """The timed runs' ms/step: how many, the median (the reported figure),
    the fastest and the slowest, and each in order."""
    return {"count": len(run_ms), "median_ms_per_step": round(statistics.median(run_ms), 5),
            "min_ms_per_step": round(min(run_ms), 5), "max_ms_per_step": round(max(run_ms), 5),
            "each_ms_per_step": [round(x, 5) for x in run_ms]}


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
    decoder_file = S.workload_decoder_file(shape, dtype, w["seed"])
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

    def timed_run():
        """One whole sequence; returns (GPU ms, tokens [stream][step], host s, enqueue s)."""
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
        enqueue = time.perf_counter() - host0
        torch.cuda.synchronize()
        host = time.perf_counter() - host0
        return start.elapsed_time(stop), ring[t:t + args.steps + 1].cpu().numpy().T, host, enqueue

    print(f"[bench] timed region: {args.runs} runs", file=sys.stderr, flush=True)
    runs = [timed_run() for _ in range(args.runs)]
    run_ms = [r[0] / args.steps for r in runs]
    ms_per_step = statistics.median(run_ms)
    gpu_ms = ms_per_step * args.steps
    tokens = runs[0][1]
    if any(not np.array_equal(r[1], tokens) for r in runs):
        print("[bench] the timed runs decoded different tokens", file=sys.stderr)
        sys.exit(3)
    median_run = min(runs, key=lambda r: abs(r[0] / args.steps - ms_per_step))
    host_s, enqueue_s = median_run[2], median_run[3]

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
        "dtype": ("f16-weights/f32" if dtype == "F16" else
                  "bf16-weights held as exact scaled fp16/f32" if decoder.product_storage == "F16" else
                  "bf16-weights/f32"),
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
        "runs": run_summary(run_ms),
        "host_seconds": round(host_s, 4),
        "host_enqueue_seconds": round(enqueue_s, 4),
    }
    print(json.dumps(line))


def encoder_flops(shape) -> float:
    """Algorithmic flops of one window: both convolutions (kernel 3), per
    layer the q/k/v/out products, fc1 and fc2, and the attention's two
    products (QK^T and PV over every head)."""
    T, d, f, L = shape.positions(), shape.width, shape.feed_forward_width, shape.layers
    conv = 2.0 * shape.input_frames * d * shape.mel_bins * 3 + 2.0 * T * d * d * 3
    layer = 4 * 2.0 * T * d * d + 2 * 2.0 * T * d * f + 2 * 2.0 * T * T * d
    return conv + L * layer


def bench_encoder(args):
    """One 30 s window through the encoder (conv stem, transformer layers,
    final LayerNorm), inputs resident in HBM; the dominant kernel, the fc1
    product on the matrix cores, timed alone on the same stream."""
    import numpy as np
    import torch
    from whispereacp_amd import synthetic as S
    from whispereacp_amd import _native as N
    from whispereacp_amd.decoder import KernelContext, to_device
    from whispereacp_amd.encoder import Encoder, EncoderWeights

    name = args.workload.split("-", 1)[1]
    dtype = ENCODER_DTYPES[name]
    shape = S.encoder_workload_shape(name)
    steps = 10 if args.steps is None else args.steps
    warmup = min(args.warmup, 3)
    print(f"[bench] generating {name} encoder weights ({dtype})", file=sys.stderr, flush=True)
    encoder_file = S.workload_encoder_file(shape, dtype, 3000)
    mel_host = S.normal_mel(shape, 3500)
    torch.cuda.set_device(0)
    mel = to_device(mel_host)
    encoder = Encoder(shape)
    weights = EncoderWeights(shape, encoder_file)
    out = torch.empty((shape.positions(), shape.width), dtype=torch.float32, device="cuda")
    for _ in range(max(1, warmup)):
        encoder.encode(mel, weights, out)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    host0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        encoder.encode(mel, weights, out)
    stop.record(stream)
    torch.cuda.synchronize()
    host_s = time.perf_counter() - host0
    ms = start.elapsed_time(stop) / steps
    flops = encoder_flops(shape)

    # The dominant kernel: fc1 of layer 0 (T x d in, f out, GELU) on the same stream.
    T, d, f = shape.positions(), shape.width, shape.feed_forward_width
    context = KernelContext(S.DecoderShape(d, shape.heads, 1, f, 16, 16, T))
    x = torch.randn((T, d), dtype=torch.float32, device="cuda")
    y = torch.empty((T, f), dtype=torch.float32, device="cuda")
    w1 = to_device(np.ascontiguousarray(encoder_file[S.encoder_layer_name(0, "fc1.weight")].data))
    b1 = to_device(encoder_file[S.encoder_layer_name(0, "fc1.bias")].floats().astype(np.float32))
    wtype = {"F16": N.WSP_F16, "BF16": N.WSP_BF16, "F32": N.WSP_F32}[dtype]
    for _ in range(3):
        context.linear(x, T, d, w1, wtype, b1, y, f, 1)
    torch.cuda.synchronize()
    launches = 50
    start.record(stream)
    for _ in range(launches):
        context.linear(x, T, d, w1, wtype, b1, y, f, 1)
    stop.record(stream)
    torch.cuda.synchronize()
    fc1_us = start.elapsed_time(stop) * 1e3 / launches
    fc1_tflops = 2.0 * T * d * f / (fc1_us * 1e-6) / 1e12
    peak = MFMA_PEAK_TFLOPS[dtype]
    context.close()

    baseline = None
    if args.cpu_budget > 0:
        print("[bench] cpu baseline (oracle encoder)", file=sys.stderr, flush=True)
        baseline = encoder_cpu_baseline(shape, encoder_file, mel_host)

    line = {
        "metric": "encoder ms per 30 s window (mel in HBM to encoded rows)",
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": steps,
        "warmup": max(1, warmup),
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("f16-weights/f32 (activations as fp16 hi/lo parts)" if dtype == "F16" else
                  "bf16-weights held as exact scaled fp16/f32 (activations as fp16 hi/lo parts)"
                  if weights.dtype == "F16" else "bf16-weights/f32 (activations as exact bf16 parts)"),
        "data": "synthetic: N(0,0.02) weights (LayerNorm gamma 1, beta 0), N(0,0.5) clipped mel",
        "config": {"workload": f"{name} encoder: {shape.mel_bins} mel bins x {shape.input_frames} frames, d_model "
                               f"{d}, {shape.heads} heads, {shape.layers} layers, ffn {f}, {T} positions, {dtype} "
                               f"projections; {steps} windows timed back to back",
                   "global_batch": 1, "seq_len": T, "parallelism": "none (one GPU)",
                   "window_tflops": round(flops / 1e12, 4),
                   "window_achieved_tflops": round(flops / (ms * 1e-3) / 1e12, 1)},
        "roofline": {"bound": "mfma", "achieved": round(fc1_tflops, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(fc1_tflops / peak, 4), "traffic": None,
                     "kernel": f"tile_product_kernel through wsp_hip_linear (fp32 rows in), fc1 shape ({T} x {d} -> "
                               f"{f}, GELU), {fc1_us:.1f} us per launch; the encoder itself runs its products "
                               f"over pre-split rows (split_product_kernel), timed in its kernel trace",
                     "flops_per_launch": 2.0 * T * d * f,
                     "note": "algorithmic flops; the matrix cores do 2x (fp16) or 3x (bf16) of them, one "
                             "product per exact 16-bit part of the fp32 activations"},
        "cpu_baseline": baseline,
        "host_seconds": round(host_s, 4),
    }
    print(json.dumps(line))


def encoder_cpu_baseline(shape, encoder_file, mel):
    """oracle_encode (double precision) on every usable core over the same
    window: the stem alone (no layers) and the stem with one layer, the whole
    encoder's time extrapolated as stem + layers x (one layer)."""
    import dataclasses
    from oracle import load_oracle
    from whispereacp_amd import synthetic as S

    host = host_description()
    cores = all_cores(host)
    oracle = load_oracle()
    oracle.set_threads(cores)
    times = []
    for layers in (0, 1):
        run = dataclasses.replace(shape, layers=layers)
        tensors = [encoder_file[n].floats() for n in S.encoder_canonical_names(layers)]
        t0 = time.perf_counter()
        oracle.encode(run, tensors, mel)
        times.append(time.perf_counter() - t0)
    stem, one = times
    estimate = stem + shape.layers * max(one - stem, 0.0)
    return {"value": round(estimate * 1e3, 1), "unit": "ms per window", "cores": cores, "kind": "port",
            "sample": f"the same window through the stem alone ({stem:.2f} s) and the stem plus one layer "
                      f"({one:.2f} s) on {cores} threads in double precision; {shape.layers} layers extrapolated",
            "host": host}


def bench_transcribe(args):
    """Whisper end to end at the tiny.en shape, the reference's own benchmark
    (Benchmark/README.md:62-106): a synthetic tiny.en directory (fp16-exact
    weights, so they load packed as the published checkpoint does), 11 s of
    audio in one window, 25 decode steps. One warm-up run, then the median of
    the timed runs; decode is the first step's submit to the last token read."""
    import statistics
    import tempfile
    import numpy as np
    import torch
    from whispereacp_amd import synthetic as S
    from whispereacp_amd.whisper import Whisper

    runs = 10 if args.steps is None else args.steps
    directory = tempfile.mkdtemp(prefix="wsp_tiny_")
    print("[bench] writing a synthetic tiny.en directory", file=sys.stderr, flush=True)
    S.tiny_en_whisper_directory(directory)
    torch.cuda.set_device(0)
    whisper = Whisper().load(directory).prepare(0)
    whisper.set_maximum_tokens(25)
    samples = S.tone_and_noise(176000)
    whisper.transcribe(samples)
    encode, decode, steps_read, tokens = [], [], [], None
    for _ in range(runs):
        tokens = whisper.transcribe(samples)
        e, d, n = whisper.timing()
        encode.append(e)
        decode.append(d)
        steps_read.append(n)
    decode_s, encode_s = statistics.median(decode), statistics.median(encode)
    steps = int(statistics.median(steps_read))
    decoder_shape = S.workload_shape("tiny.en")
    bytes_per_step = sum(step_bytes(decoder_shape, 2, p) for p in range(2, 2 + steps)) / max(steps, 1)
    achieved = bytes_per_step / (decode_s / max(steps, 1)) / 1e9

    baseline = None
    if args.cpu_budget > 0:
        print("[bench] cpu baseline (oracle chain)", file=sys.stderr, flush=True)
        baseline = transcribe_cpu_baseline(directory, samples, whisper, tokens)

    line = {
        "metric": "tiny.en transcribe: decode seconds for 25 steps (first submit to last token read), median",
        "value": round(decode_s, 6),
        "unit": "s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 1,
        "ms_per_step": round(decode_s / max(steps, 1) * 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(decode_s / REFERENCE_TINY_DECODE_S, 4),
        "dtype": "f16-weights/f32",
        "data": "synthetic: fp16-exact N(0,0.02) weights, tone-and-noise audio (11 s); the published figure is "
                "real tiny.en weights on jfk.wav (same shapes, same step count)",
        "config": {"workload": "tiny.en Whisper: mel (30 s, 80 bands) -> encoder (4 layers, d 384) -> greedy "
                               "decoder (4 layers, vocab 51864, 25 steps) -> text",
                   "encode_s_median": round(encode_s, 6), "runs": runs, "tokens": len(tokens),
                   "global_batch": 1, "seq_len": 2 + steps, "parallelism": "none (one GPU)",
                   "baseline": f"{REFERENCE_TINY_DECODE_S} s, Apple M5 Max (README.md:44-53)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode steps (persistent step kernel), host loop included",
                     "bytes_per_step": round(bytes_per_step)},
        "cpu_baseline": baseline,
    }
    print(json.dumps(line))


def transcribe_cpu_baseline(directory, samples, whisper, gpu_tokens):
    """The same chain on the oracle (mel, encoder, KV-cached decoder under the
    two masks) on every usable core: seconds for the encode and for the
    decode's steps, and whether its tokens match the GPU's."""
    import numpy as np
    from oracle import load_oracle
    from whispereacp_amd import synthetic as S
    from whispereacp_amd.decoder import SafeTensorsFile

    host = host_description()
    cores = all_cores(host)
    oracle = load_oracle()
    oracle.set_threads(cores)
    file = SafeTensorsFile(os.path.join(directory, "model.safetensors"))
    sizes = {n: s for n, _, s, _ in file.tensors()}

    def floats(n):
        return file.read_floats(n, int(np.prod(sizes[n]))).reshape(sizes[n])

    encoder, decoder, mel_shape = S.encoder_workload_shape("tiny.en"), S.workload_shape("tiny.en"), S.MelShape()
    window = np.zeros(mel_shape.sample_count, dtype=np.float32)
    window[:len(samples)] = samples
    t0 = time.perf_counter()
    mel = oracle.mel_spectrogram(window, S.triangular_filters(80, mel_shape.bin_count), mel_shape.fft_length,
                                 mel_shape.hop_length, mel_shape.frame_count)
    rows = oracle.encode(encoder, [floats(n) for n in S.encoder_canonical_names(encoder.layers)],
                         mel.astype(np.float32))
    encode_s = time.perf_counter() - t0
    first, later = whisper.masks(decoder.vocabulary_size)
    session = oracle.session(decoder, [floats(n) for n in S.canonical_names(decoder.layers)])
    t0 = time.perf_counter()
    session.begin(rows.astype(np.float32))
    _, logits = session.step(whisper.prompt())
    tokens = [int(np.argmax(np.where(first != 0, -np.inf, logits[-1])))]
    for _ in range(len(gpu_tokens) - 1):
        _, logits = session.step([tokens[-1]])
        tokens.append(int(np.argmax(np.where(later != 0, -np.inf, logits[0]))))
    decode_s = time.perf_counter() - t0
    return {"value": round(decode_s, 3), "unit": "s (decode, 25 steps)", "cores": cores, "kind": "port",
            "sample": f"the whole run: oracle mel + encoder {encode_s:.2f} s, then begin_sequence and "
                      f"{len(tokens)} decode steps in double precision on {cores} threads",
            "encode_s": round(encode_s, 3), "tokens_match": tokens == list(gpu_tokens), "host": host}


if __name__ == "__main__":
    main()
