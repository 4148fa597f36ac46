"""Per-phase critical path of the persistent decode step.

    python -m cq35.phase_trace [--config qwen36-35b-a3b] [--context 512]
                               [--long 0] [--steps 8] [--build]

Covers the MoE step (k_decode_step) and the dense step (k_dense_step).
Uses the phase-trace build of the library (libcq35_trace.so, compiled with
-DCQ35_PHASE_TRACE; --build or a missing file compiles it), decodes `steps`
tokens after a `context`-token prompt (or, with --long N, from a seeded
state of N cached positions) and prints a markdown table for the last step:
per phase of a linear (DeltaNet) and a full-attention layer, averaged over
the layers of that kind,
  - critical path: the last block's completion of the phase minus the last
    block's completion of the phase before it in the chain;
  - inputs in: the last block's end of polling for the phase's inputs minus
    that previous completion (exchange latency plus any wait behind the
    phase's own loads);
  - the HBM floor of the phase's algorithmic bytes at 8 TB/s;
and for full layers the values phase's busy time per role, or, when the
step ran split-K attention (more keys than the session's split threshold),
the flash phase's time per stage. Stamps are s_memrealtime (100 MHz, 10 ns).
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys

import numpy as np

from . import _build, _lib
from .config import derived, is_full, preset

TRACE_LAYER_SLOTS = 32  # mega.h kTraceLayerSlots
TRACE_LAYERS = 48
TRACE_HEAD = TRACE_LAYERS * TRACE_LAYER_SLOTS
TRACE_START = TRACE_HEAD + 1
TICK_US = 0.01
HBM_GBS = 8000.0

LINEAR = ["project", "delta", None, "outproj", "router + shared", "select + gate/up", "down"]
# mega.h TraceMark: (slot, phase index, label)
MARKS = [(20, 0, "input row normalised"), (21, 1, "convolution done"), (22, 1, "L2 norms and gates done"),
         (23, 1, "state update done"), (29, 3, "outputs computed"), (24, 4, "post-mixer row normalised"),
         (25, 5, "experts selected"), (26, 5, "outputs stored"), (27, 6, "staged weights and inputs in"),
         (28, 6, "outputs stored")]
FULL = ["project", "scores", "values", "outproj", "router + shared", "select + gate/up", "down"]
# dense_step.h (k_dense_step): p0 project, p1 delta or scores, p3 softmax +
# context, p4 output projection, p5 gate/up, p6 down
DENSE_LINEAR = ["project", "delta", None, None, "outproj", "gate/up", "down"]
DENSE_FULL = ["project", "scores", None, "softmax + context", "outproj", "gate/up", "down"]
DENSE_MARKS = [(20, 0, "input row normalised"), (21, 1, "convolution done"), (22, 1, "L2 norms and gates done"),
               (23, 1, "state update done"), (29, 4, "outputs computed"), (24, 5, "post-mixer row normalised"),
               (26, 5, "outputs stored")]
# full layers of the dense step reuse slots 21-23 inside the attention phases
DENSE_MARKS_FULL = [(20, 0, "input row normalised"), (21, 1, "heads prepared"), (22, 3, "softmax done"),
                    (23, 3, "chains done"), (29, 4, "outputs computed"), (24, 5, "post-mixer row normalised"),
                    (26, 5, "outputs stored")]


def phase_bytes(cfg: dict, keys: int) -> dict:
    d = derived(cfg)
    H, VH, VD, KD = cfg["hidden"], cfg["value_heads"], cfg["value_dim"], cfg["key_dim"]
    K, I, SI, E = cfg["top_k"], cfg["intermediate"], cfg["shared_intermediate"], cfg["experts"]
    if not E:
        return {
            ("lin", "project"): (d["qkv"] + d["value_size"] + 2 * VH) * H * 2,
            ("full", "project"): (2 * d["query_size"] + 2 * d["kvs"]) * H * 2,
            ("lin", "delta"): 2 * VH * VD * KD * 2 + 4 * d["qkv"] * 2,
            ("full", "scores"): keys * d["kvs"] * 2,
            ("full", "softmax + context"): keys * d["kvs"] * 2,
            ("lin", "outproj"): H * d["value_size"] * 2,
            ("full", "outproj"): H * d["query_size"] * 2,
            ("gate/up",): 2 * I * H * 2,
            ("down",): I * H * 2,
        }
    # MoE step: a linear layer's z rows are computed during the delta phase
    return {
        ("lin", "project"): (d["qkv"] + 2 * VH) * H * 2,
        ("full", "project"): (2 * d["query_size"] + 2 * d["kvs"]) * H * 2,
        ("lin", "delta"): 2 * VH * VD * KD * 2 + 4 * d["qkv"] * 2 + d["value_size"] * H * 2,
        ("full", "scores"): keys * d["kvs"] * 2,
        ("full", "values"): keys * d["kvs"] * 2,
        ("lin", "outproj"): H * d["value_size"] * 2,
        ("full", "outproj"): H * d["query_size"] * 2,
        ("router + shared",): (E + 1) * H * 4 + 2 * SI * H * 2,
        ("select + gate/up",): 2 * K * I * H * 2,
        ("down",): (K * I + SI) * H * 2,
    }


def floor_us(pb: dict, kind: str, name: str) -> float:
    b = pb.get((kind, name), pb.get((name,), 0))
    return b / (HBM_GBS * 1e3)


def analyse(trace: np.ndarray, cfg: dict, keys: int, flash: bool = False) -> str:
    L = cfg["layers"]
    start = trace[:, TRACE_START][trace[:, TRACE_START] > 0].min()
    pb = phase_bytes(cfg, keys)
    rows = {"lin": {}, "full": {}}
    timeline = {"lin": {}, "full": {}}
    per_layer = []
    prev_done = start
    roles = []
    dense = not cfg.get("experts")
    lin_names, full_names = (DENSE_LINEAR, DENSE_FULL) if dense else (LINEAR, FULL)
    for l in range(L):
        tb = l * TRACE_LAYER_SLOTS
        kind = "full" if is_full(cfg, l) else "lin"
        names = full_names if kind == "full" else lin_names
        layer_start = prev_done
        tl = timeline[kind]
        for p, name in enumerate(names):
            if name is None:
                continue
            done = trace[:, tb + 2 * p].max()
            polled = trace[:, tb + 2 * p + 1]
            polled = polled[polled > 0]
            inputs = (polled.max() - prev_done) if polled.size else 0
            if polled.size:
                tl.setdefault((p, 0, name + ": inputs in"), []).append((polled.max() - layer_start) * TICK_US)
            for slot, mp, label in (MARKS if not dense else DENSE_MARKS_FULL if kind == "full" else DENSE_MARKS):
                if mp == p:
                    v = trace[:, tb + slot]
                    v = v[v > 0]
                    if v.size:
                        tl.setdefault((p, slot, name + ": " + label), []).append((v.max() - layer_start) * TICK_US)
            tl.setdefault((p, 99, name + ": done"), []).append((done - layer_start) * TICK_US)
            r = rows[kind].setdefault(name, [0.0, 0.0, 0])
            r[0] += (done - prev_done) * TICK_US
            r[1] += inputs * TICK_US
            r[2] += 1
            prev_done = done
        per_layer.append((l, kind, (prev_done - layer_start) * TICK_US))
        if kind == "full" and not dense:
            if flash:
                busy = trace[:, tb + 14:tb + 19].astype(np.float64)
                busy = np.concatenate([busy[:, :4].mean(axis=0) * TICK_US, busy[:, :4].max(axis=0) * TICK_US,
                                       [busy[:, 4].sum()]])
            else:
                busy = trace[:, tb + 14:tb + 18].astype(np.float64).mean(axis=0) * TICK_US
            roles.append(busy)
    head = (trace[:, TRACE_HEAD].max() - prev_done) * TICK_US
    total = (trace[:, TRACE_HEAD].max() - start) * TICK_US
    out = []
    for kind, names, label in [("lin", lin_names, "linear (DeltaNet) layer"), ("full", full_names, "full-attention layer")]:
        n = sum(1 for _, k, _ in per_layer if k == kind)
        if n == 0:
            continue
        out.append(f"\n**{label}** (mean of {n} layers)\n")
        out.append("| phase | critical path (us) | inputs in (us) | HBM floor at 8 TB/s (us) |")
        out.append("|---|---|---|---|")
        tot = 0.0
        for name in names:
            if name is None or name not in rows[kind]:
                continue
            c, i, cnt = rows[kind][name]
            tot += c / cnt
            out.append(f"| {name} | {c / cnt:.2f} | {i / cnt:.2f} | {floor_us(pb, kind, name):.2f} |")
        out.append(f"| **layer** | **{tot:.2f}** | | |")
        out.append(f"\n*{label} timeline* (last wave to reach the point, us from the layer's start, mean)\n")
        out.append("| point | us |")
        out.append("|---|---|")
        for key in sorted(timeline[kind]):
            out.append(f"| {key[2]} | {np.mean(timeline[kind][key]):.2f} |")
    if roles and flash:
        b = np.mean(roles, axis=0)
        out.append("\n**flash phase, time per stage** (per full layer, us; mean over blocks / slowest block; "
                   f"{b[8]:.0f} items): prepare {b[0]:.2f} / {b[4]:.2f}, scores {b[1]:.2f} / {b[5]:.2f}, "
                   f"scan {b[2]:.2f} / {b[6]:.2f}, values and partials {b[3]:.2f} / {b[7]:.2f}\n")
    elif roles:
        b = np.mean(roles, axis=0)
        out.append("\n**values phase, busy time per role** (mean per block and full layer, us): "
                   f"scan {b[0]:.2f}, products (4 waves, summed) {b[1]:.2f}, channel chains {b[2]:.2f}, "
                   f"denominator chain {b[3]:.2f}\n")
    out.append(f"\nhead (final norm + vocabulary + argmax): {head:.2f} us "
               f"(HBM floor {cfg['vocab'] * cfg['hidden'] * 2 / (HBM_GBS * 1e3):.2f} us); "
               f"step from first stamp to head end: {total:.1f} us\n")
    return "\n".join(out)


def seeded_state(cfg: dict, capacity: int, position: int, seed: int) -> np.ndarray:
    """BF16 state like the long-context benchmark's: K/V rows of positions
    below `position` ~ 0.1 N(0,1), conv history ~ 0.1 N(0,1), DeltaNet state
    ~ N(0,1) (numpy's generator; the timing does not depend on the values)."""
    d = derived(cfg)
    L, kvs = cfg["layers"], d["kvs"]
    lin = d["conv"] + d["recurrent"]
    rng = np.random.default_rng(seed)
    out = np.zeros(capacity * L * 2 * kvs + L * lin, dtype=np.float32)
    kv = out[:capacity * L * 2 * kvs].reshape(L * 2, capacity, kvs)
    for r in range(L * 2):
        kv[r, :position] = rng.standard_normal((position, kvs), dtype=np.float32) * 0.1
    tail = out[capacity * L * 2 * kvs:].reshape(L, lin)
    tail[:, :d["conv"]] = rng.standard_normal((L, d["conv"]), dtype=np.float32) * 0.1
    tail[:, d["conv"]:] = rng.standard_normal((L, lin - d["conv"]), dtype=np.float32)
    return (out.view(np.uint32) >> 16).astype(np.uint16)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--config", default="qwen36-35b-a3b")
    ap.add_argument("--context", type=int, default=512)
    ap.add_argument("--long", type=int, default=0, help="decode from a seeded state of this many positions")
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--build", action="store_true")
    ap.add_argument("--dump", default="", help="also save the raw [blocks][slots] stamps (numpy .npy)")
    args = ap.parse_args()
    if args.build or not os.path.exists(_build.TRACE_LIBRARY):
        _build.build(trace=True)
    _lib.LIBRARY = os.environ.get("CQ35_LIBRARY") or _build.TRACE_LIBRARY
    from . import model as cq
    cfg = preset(args.config)
    m = cq.Model.synthetic(cfg, seed=0)
    if args.long:
        cap = args.long + args.steps + 4
        s = m.session(cap)
        s.import_state(0, seeded_state(cfg, cap, args.long, 101))
        s.position = args.long
        nxt = 1
    else:
        cap = args.context + args.steps + 4
        s = m.session(cap)
        nxt = s.append_next_token([(7 * i) % cfg["vocab"] for i in range(args.context)])
    if not s.persistent:
        print("this shape has no persistent decode step", file=sys.stderr)
        return 2
    for _ in range(args.steps):
        nxt = s.decode_next_token(nxt)
    lib = _lib.load()
    slots, blocks = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(lib.cq35_session_phase_trace(s._h, None, 0, ctypes.byref(slots), ctypes.byref(blocks)))
    n, blocks = slots.value, blocks.value
    buf = np.zeros(blocks * n, dtype=np.uint64)
    _lib.check(lib.cq35_session_phase_trace(s._h, buf.ctypes.data, buf.size, ctypes.byref(slots),
                                            ctypes.byref(ctypes.c_int64())))
    trace = buf.reshape(blocks, n).astype(np.int64)
    if args.dump:
        np.save(args.dump, trace)
    keys = (args.long or args.context) + args.steps
    split = s.attention_split
    flash = split > 0 and keys > split
    print(f"{args.config}, {blocks} blocks, {'long ' + str(args.long) if args.long else 'context ' + str(args.context)}"
          f" + {args.steps} steps (last step traced, about {keys} keys)")
    print(analyse(trace, cfg, keys, flash))
    return 0


if __name__ == "__main__":
    sys.exit(main())
