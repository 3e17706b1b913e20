"""Per-layer timeline of the persistent single-token step.

The timeline variant of the library (build.build_timeline(): the step kernel
built with WSP_STEP_TIMELINE) stamps the GPU's 100 MHz real-time clock at every
phase boundary of every workgroup. This tool runs the small decode workload
(d 768, 12 heads, 12 layers, vocab 51865, fp16 weights, 1500 cross rows, the
4-token prefix then single-token greedy steps) on that variant, records the
stamps of a sample of steps spread over the sequence, and prints a markdown
table: for each hand-over the median consumer's arrival less the last
producer's finish, and for each phase the median workgroup's time from its
input's arrival to the end of its stores and of the next phase's prefetch
issue, averaged over the layers and the sampled steps.

    python -m whispereacp_amd.step_timeline --build     # on the build host
    python -m whispereacp_amd.step_timeline             # on the GPU
    python -m whispereacp_amd.step_timeline --tokens 4  # one 4-token launch instead

With --tokens N the tool records launches of the multi-token kernel (N tokens
at position 0, without the fused argmax) instead of single-token steps.

The stamps cost a few instructions each, so the step runs a little slower
under this variant than in the product build; the table is for the shape of
the chain, the product build's kernel trace for its length.
"""

from __future__ import annotations

import argparse
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Stamp events (step_kernel.hip STEP_STAMP(event, layer)).
H_IN, QKV_DONE, SELF_IN, OUT_DONE, H2_IN, XQ_DONE, XQ_IN, XPART_DONE = 0, 1, 2, 3, 4, 5, 6, 7
XATTN_IN, XOUT_DONE, H3_IN, FC1_DONE, FF_IN, FC2_DONE = 8, 9, 10, 11, 12, 13
HEAD_QKV_IN, HEAD_SELF_DONE, HEAD_XPART_IN, HEAD_COMBINE_DONE = 14, 15, 16, 17
FINAL_IN, LOGITS_DONE, ARGMAX_DONE, TABLE_DONE = 18, 19, 20, 21
# Marks inside the phases: attention (after the scores' maximum, after the
# weighted sums' folds, after the barrier) and each projection (after the dot
# products, after the partial sums' barrier and the stores).
ATT_MAX, ATT_FOLDED, ATT_BARRIER = 22, 23, 24
LOGITS_ALL, CANDIDATES_IN = 37, 38 # every row group of a workgroup done; the fold's poll done
QKV_DOT, OUT_DOT, XQ_DOT, XOUT_DOT, FC1_DOT, FC2_DOT = 25, 27, 29, 31, 33, 35
EVENTS, LAYER_SLOTS = 40, 33
TICK_US = 0.01  # 100 MHz

# (label, consumer event, consumer role, producer event, producer role, layer offset of the producer)
HANDOVERS = [
    ("h (previous layer) -> row groups", H_IN, "row", FC2_DONE, "row", -1),
    ("q/k/v -> head groups", HEAD_QKV_IN, "attend", QKV_DONE, "row", 0),
    ("self rows -> row groups", SELF_IN, "row", HEAD_SELF_DONE, "attend", 0),
    ("h2 -> row groups", H2_IN, "row", OUT_DONE, "row", 0),
    ("cross q -> cross tasks", XQ_IN, "task", XQ_DONE, "row", 0),
    ("cross partials -> head groups", HEAD_XPART_IN, "combine", XPART_DONE, "task", 0),
    ("cross rows -> row groups", XATTN_IN, "row", HEAD_COMBINE_DONE, "combine", 0),
    ("h3 -> row groups", H3_IN, "row", XOUT_DONE, "row", 0),
    ("fc1 output -> row groups", FF_IN, "row", FC1_DONE, "row", 0),
]
# (label, start event, end event, role)
PHASES = [
    ("LN1 + q/k/v", H_IN, QKV_DONE, "row"),
    ("self attention", HEAD_QKV_IN, HEAD_SELF_DONE, "attend"),
    ("out-projection", SELF_IN, OUT_DONE, "row"),
    ("LN2 + cross q", H2_IN, XQ_DONE, "row"),
    ("cross attention chunk", XQ_IN, XPART_DONE, "task"),
    ("cross combine", HEAD_XPART_IN, HEAD_COMBINE_DONE, "combine"),
    ("cross out-projection", XATTN_IN, XOUT_DONE, "row"),
    ("LN3 + fc1", H3_IN, FC1_DONE, "row"),
    ("fc2", FF_IN, FC2_DONE, "row"),
]


# (phase, role, [(part, start event, end event)]). The LayerNorms are folded
# into the projections that consume them: their statistics come from the
# polls, so those phases start with the dot products.
INSIDE = [
    ("LN1 + q/k/v", "row", [("statistics, dot products", H_IN, QKV_DOT),
                            ("partial sums, barrier, stores", QKV_DOT, QKV_DOT + 1),
                            ("next weights issued", QKV_DOT + 1, QKV_DONE)]),
    ("self attention", "attend", [("scores and maximum", HEAD_QKV_IN, ATT_MAX), ("weights, sums, folds", ATT_MAX, ATT_FOLDED),
                                  ("LDS and barrier", ATT_FOLDED, ATT_BARRIER), ("wave combine, stores", ATT_BARRIER,
                                                                                 HEAD_SELF_DONE)]),
    ("out-projection", "row", [("dot products", SELF_IN, OUT_DOT), ("partial sums, barrier, stores", OUT_DOT, OUT_DOT + 1),
                               ("next weights issued", OUT_DOT + 1, OUT_DONE)]),
    ("LN2 + cross q", "row", [("statistics, dot products", H2_IN, XQ_DOT),
                              ("partial sums, barrier, stores", XQ_DOT, XQ_DOT + 1),
                              ("next weights issued", XQ_DOT + 1, XQ_DONE)]),
    ("cross attention chunk", "task", [("scores and maximum", XQ_IN, ATT_MAX), ("weights, sums, folds", ATT_MAX, ATT_FOLDED),
                                       ("LDS and barrier", ATT_FOLDED, ATT_BARRIER),
                                       ("wave combine, stores", ATT_BARRIER, XPART_DONE)]),
    ("cross out-projection", "row", [("dot products", XATTN_IN, XOUT_DOT),
                                     ("partial sums, barrier, stores", XOUT_DOT, XOUT_DOT + 1),
                                     ("next weights issued", XOUT_DOT + 1, XOUT_DONE)]),
    ("LN3 + fc1", "row", [("statistics, dot products", H3_IN, FC1_DOT),
                          ("partial sums, barrier, stores", FC1_DOT, FC1_DOT + 1),
                          ("next weights issued", FC1_DOT + 1, FC1_DONE)]),
    ("fc2", "row", [("dot products", FF_IN, FC2_DOT), ("partial sums, barrier, stores", FC2_DOT, FC2_DOT + 1),
                    ("next weights issued", FC2_DOT + 1, FC2_DONE)]),
]


def roles(stamps, layers):
    """Workgroup indices by role, read from which events each one stamped."""
    import numpy as np
    row = np.nonzero(stamps[:, FC2_DONE, 0] != 0)[0]
    attend = np.nonzero(stamps[:, HEAD_SELF_DONE, 0] != 0)[0]
    combine = np.nonzero(stamps[:, HEAD_COMBINE_DONE, 0] != 0)[0]
    task = np.intersect1d(np.nonzero(stamps[:, XQ_IN, 0] != 0)[0], row)  # stamped on their first task
    return {"row": row, "attend": attend, "combine": combine, "task": task}


def step_table(stamps, layers):
    """Per-layer hand-over and phase times (microseconds) of one step's stamps
    [workgroups][events][layer slots]."""
    import numpy as np
    r = roles(stamps, layers)
    t = stamps.astype(np.float64) * TICK_US
    hand = {label: [] for label, *_ in HANDOVERS}
    phase = {label: [] for label, *_ in PHASES}
    layer_time = []
    for l in range(layers):
        for label, ce, crole, pe, prole, off in HANDOVERS:
            pl = l + off
            if pl < 0:
                continue
            hand[label].append(np.median(t[r[crole], ce, l]) - np.max(t[r[prole], pe, pl]))
        for label, se, ee, role in PHASES:
            phase[label].append(np.median(t[r[role], ee, l] - t[r[role], se, l]))
        if l > 0:
            layer_time.append(np.median(t[r["row"], FC2_DONE, l]) - np.median(t[r["row"], FC2_DONE, l - 1]))
    everyone = np.arange(stamps.shape[0])
    tail = {
        "final h -> every workgroup": np.median(t[everyone, FINAL_IN, 0]) - np.max(t[r["row"], FC2_DONE, layers - 1]),
        "final LayerNorm + tied logits": np.median(t[everyone, LOGITS_DONE, 0] - t[everyone, FINAL_IN, 0]),
        "slowest logits workgroup": np.max(t[everyone, LOGITS_DONE, 0] - t[everyone, FINAL_IN, 0]),
        "row groups' imbalance (last row group of a workgroup, median)": np.median(
            t[everyone, LOGITS_ALL, 0] - t[everyone, LOGITS_DONE, 0]),
    }
    start = np.median(t[r["row"], TABLE_DONE, 0])
    if np.max(stamps[:, ARGMAX_DONE, 0]) != 0:
        tail["last workgroup done -> fold sees every candidate"] = (float(np.max(t[:, CANDIDATES_IN, 0]))
                                                                   - np.max(t[everyone, LOGITS_ALL, 0]))
        tail["fold -> token written"] = float(np.max(t[:, ARGMAX_DONE, 0])) - float(np.max(t[:, CANDIDATES_IN, 0]))
        tail["argmax fold (last candidate -> token)"] = (float(np.max(t[:, ARGMAX_DONE, 0]))
                                                         - np.max(t[everyone, LOGITS_DONE, 0]))
        whole = float(np.max(t[:, ARGMAX_DONE, 0])) - start
    else:
        # A step without the fused argmax (a multi-token step) ends with its logits.
        whole = float(np.max(t[everyone, LOGITS_ALL, 0])) - start
    inside = {}
    for label, role, parts in INSIDE:
        for part, se, ee in parts:
            # (a part the kernel does not mark, e.g. inside a multi-token
            # cross-attention chunk, is left out)
            if np.all(stamps[r[role], se, :layers] != 0) and np.all(stamps[r[role], ee, :layers] != 0):
                inside[(label, part)] = float(np.mean([np.median(t[r[role], ee, l] - t[r[role], se, l])
                                                       for l in range(layers)]))
    return ({k: float(np.mean(v)) for k, v in hand.items()}, {k: float(np.mean(v)) for k, v in phase.items()},
            float(np.mean(layer_time)), {k: float(v) for k, v in tail.items()}, whole,
            {k: len(v) for k, v in r.items()}, inside)


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--build", action="store_true", help="build the timeline variant of the library and exit")
    parser.add_argument("--samples", type=int, default=16, help="steps of the sequence whose stamps are recorded")
    parser.add_argument("--steps", type=int, default=224, help="single-token steps in the sequence")
    parser.add_argument("--tokens", type=int, default=0,
                        help="record instead one multi-token step of this many tokens (at most 4) at position 0")
    args = parser.parse_args()

    sys.path.insert(0, ROOT)
    from whispereacp_amd import build as B
    if args.build:
        B.build_timeline()
        return
    if not os.path.exists(B.TIMELINE_LIBRARY):
        sys.exit(f"the timeline variant is not built ({B.TIMELINE_LIBRARY}); run with --build first")
    os.environ["WSP_LIBRARY"] = B.TIMELINE_LIBRARY

    import ctypes

    import numpy as np
    import torch
    from whispereacp_amd import _native as N
    from whispereacp_amd import synthetic as S
    from whispereacp_amd.decoder import Decoder, to_device

    lib = N.load()
    set_timeline = lib.wsp_step_timeline
    set_timeline.restype = None
    set_timeline.argtypes = [ctypes.c_void_p]

    shape = S.workload_shape("small")
    w = S.WORKLOADS["small"]
    decoder_file = S.workload_decoder_file(shape, w["dtype"], w["seed"])
    encoder = S.normal_encoder_output(shape.cross_positions, shape.width, 7)
    torch.cuda.set_device(0)
    decoder = Decoder(shape, decoder_file, packing="ExactHalf")
    assert decoder.uses_persistent_step, "the small shape takes the persistent step"
    prompt = S.SOT_PREFIX[shape.vocabulary_size]
    V, base = shape.vocabulary_size, len(prompt)
    workgroups = torch.cuda.get_device_properties(0).multi_processor_count
    stamps = torch.zeros((workgroups, EVENTS, LAYER_SLOTS), dtype=torch.int64, device="cuda")
    slots = torch.zeros(shape.max_positions + 1, dtype=torch.int32, device="cuda")
    slots[:base] = torch.tensor(prompt, dtype=torch.int32, device="cuda")
    prompt_logits = torch.empty((base, V), dtype=torch.float32, device="cuda")
    logits = torch.empty((1, V), dtype=torch.float32, device="cuda")

    results = []
    if args.tokens:
        # Launches of args.tokens tokens at position 0, each recorded alone.
        n = args.tokens
        ids = torch.arange(1, n + 1, dtype=torch.int32, device="cuda")
        out = torch.empty((n, V), dtype=torch.float32, device="cuda")
        for _ in range(args.samples):
            decoder.begin_sequence(to_device(encoder))
            torch.cuda.synchronize()
            stamps.zero_()
            set_timeline(stamps.data_ptr())
            decoder.step(ids, n, out)
            torch.cuda.synchronize()
            set_timeline(None)
            results.append(step_table(stamps.cpu().numpy(), shape.layers))
        what = f"{n}-token launches at position 0, {len(results)} sampled"
    else:
        decoder.begin_sequence(to_device(encoder))
        decoder.step(slots[:base], base, prompt_logits)
        decoder.argmax(prompt_logits[-1:], 1, V, None, slots[base:base + 1])
        sampled = sorted({int((i + 0.5) * args.steps / args.samples) for i in range(args.samples)})
        for j in range(1, args.steps + 1):
            take = (j - 1) in sampled
            if take:
                torch.cuda.synchronize()
                stamps.zero_()
                set_timeline(stamps.data_ptr())
            decoder.step_and_sample(slots[base + j - 1:base + j], logits, None, slots[base + j:base + j + 1])
            if take:
                torch.cuda.synchronize()
                set_timeline(None)
                results.append(step_table(stamps.cpu().numpy(), shape.layers))
        positions = [base + j for j in sampled]
        what = f"{len(results)} steps sampled at positions {positions[0]}..{positions[-1]}"
    assert decoder.device_status() == 0, "the step's watchdog tripped"

    hand = {k: float(np.mean([r[0][k] for r in results])) for k in results[0][0]}
    phase = {k: float(np.mean([r[1][k] for r in results])) for k in results[0][1]}
    layer = float(np.mean([r[2] for r in results]))
    tail = {k: float(np.mean([r[3][k] for r in results])) for k in results[0][3]}
    whole = float(np.mean([r[4] for r in results]))
    counts = results[0][5]

    print(f"Small decoder step on the timeline build, {what}; {workgroups} workgroups: {counts['row']} row groups "
          f"({counts['task']} with a cross-attention task), {counts['attend']} attending head groups, "
          f"{counts['combine']} combining. Times in microseconds, averaged over the layers and the sampled "
          f"steps.\n")
    print("| Hand-over (median consumer - last producer) | us | Phase (median workgroup) | us |")
    print("|---|---|---|---|")
    for (hl, hv), (pl, pv) in zip(hand.items(), phase.items()):
        print(f"| {hl} | {hv:.2f} | {pl} | {pv:.2f} |")
    print(f"| **sum of hand-overs** | **{sum(hand.values()):.2f}** | **sum of phases** | "
          f"**{sum(phase.values()):.2f}** |")
    print()
    print(f"Layer (median row group's fc2 finish to the next layer's): {layer:.2f} us; the rest of a layer "
          f"beyond the listed hand-overs and phases is producer skew: "
          f"{layer - sum(hand.values()) - sum(phase.values()):.2f} us.\n")
    print("| After the last layer | us |")
    print("|---|---|")
    for k, v in tail.items():
        print(f"| {k} | {v:.2f} |")
    end = "token written" if not args.tokens else "last logits row written"
    print(f"\nWhole step (layer table loaded -> {end}), timeline build: {whole:.1f} us.")
    inside = {k: float(np.mean([r[6][k] for r in results])) for k in results[0][6]}
    print("\nInside the phases (median workgroup of the phase's role, us):\n")
    print("| Phase | Part | us |")
    print("|---|---|---|")
    for (label, part), v in inside.items():
        print(f"| {label} | {part} | {v:.2f} |")


if __name__ == "__main__":
    main()
