#!/usr/bin/env python3
"""Batch-1 decode benchmark of the Qwen3.5/3.6 token loop on one MI355X.

Mirrors the reference's `--bench --tg K --tg-context C` protocol
(src/main.rs:393-445): a fresh session, the C-token synthetic prompt
(LCG ids, src/main.rs:447-457) appended as one batched call (one token per
call with --prompt-per-token), W untimed decode
steps, then K timed greedy `decode_next_token` steps, each ending with the
8-byte token readback and a stream synchronisation. Defaults are the 35B-A3B
configuration: 512-token prompt, 512 greedy decode steps (context 512-1024). Weights are random-init BF16
generated on the device (no checkpoint). One JSON line on stdout.

The CPU baseline is the C restatement (oracle/) on the same shape, timed on
the host's cores over a bounded sample, with its greedy tokens compared to
the GPU's on the same prompt.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "catena-models_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def synthetic_tokens(count: int, vocab: int) -> list[int]:
    """src/main.rs:447-457."""
    state = 0x9E3779B97F4A7C15
    out = []
    for _ in range(count):
        state = (state * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        out.append(state % vocab)
    return out


def device_sync():
    try:
        ctypes.CDLL("libamdhip64.so").hipDeviceSynchronize()
    except OSError:
        pass


def copy_probe(megabytes: int) -> None:
    """One device-to-device copy of a known size (the runtime's copy kernel),
    so hardware-counter passes can scale FETCH_SIZE / WRITE_SIZE to bytes."""
    hip = ctypes.CDLL("libamdhip64.so")
    n = megabytes << 20
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(src), ctypes.c_size_t(n)) or hip.hipMalloc(ctypes.byref(dst), ctypes.c_size_t(n)):
        raise RuntimeError("hipMalloc failed for the copy probe")
    hip.hipMemset(src, 0x3C, ctypes.c_size_t(n))
    hip.hipMemcpy(dst, src, ctypes.c_size_t(n), 3)  # hipMemcpyDeviceToDevice
    hip.hipDeviceSynchronize()
    hip.hipFree(src)
    hip.hipFree(dst)
    log(f"copy probe: {megabytes} MiB device-to-device")


def copy_ceiling(mib: int = 1024, reps: int = 10) -> dict:
    """Measured device-copy ceiling: a `mib` MiB device-to-device copy
    (the runtime's copy kernel) timed with HIP events, `reps` times; the
    best rate counts read + write bytes. The practical HBM ceiling next to
    the nominal 8 TB/s."""
    hip = ctypes.CDLL("libamdhip64.so")
    n = mib << 20
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(src), ctypes.c_size_t(n)) or hip.hipMalloc(ctypes.byref(dst), ctypes.c_size_t(n)):
        raise RuntimeError("hipMalloc failed for the copy ceiling")
    try:
        hip.hipMemset(src, 0x3C, ctypes.c_size_t(n))
        e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
        hip.hipEventCreate(ctypes.byref(e0))
        hip.hipEventCreate(ctypes.byref(e1))
        best = None
        for i in range(reps + 1):
            hip.hipEventRecord(e0, None)
            if hip.hipMemcpyAsync(dst, src, ctypes.c_size_t(n), 3, None):  # hipMemcpyDeviceToDevice
                raise RuntimeError("device copy failed")
            hip.hipEventRecord(e1, None)
            hip.hipEventSynchronize(e1)
            ms = ctypes.c_float()
            hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1)
            if i > 0 and (best is None or ms.value < best):  # the first copy is a warm-up
                best = ms.value
        hip.hipEventDestroy(e0)
        hip.hipEventDestroy(e1)
    finally:
        hip.hipDeviceSynchronize()
        hip.hipFree(src)
        hip.hipFree(dst)
    gbs = 2 * n / (best / 1e3) / 1e9
    log(f"copy ceiling: {mib} MiB device-to-device, {gbs:.0f} GB/s (read + write, best of {reps})")
    return dict(gbs=round(gbs, 1), bytes=2 * n, ms=round(best, 4), reps=reps,
                method=f"hipMemcpyAsync device-to-device of {mib} MiB, HIP events, best of {reps}")


def kernel_bytes(cfg: dict, context: int) -> dict:
    """Algorithmic HBM bytes per launch of each streaming kernel class."""
    import cq35
    d = cq35.derived(cfg)
    H, V = cfg["hidden"], cfg["vocab"]
    full = len(d["full_layers"])
    lin = cfg["layers"] - full
    lin_rows = d["qkv"] + d["value_size"] + 2 * cfg["value_heads"]
    full_rows = 2 * d["query_size"] + 2 * d["kvs"]
    out = {
        "project": ((lin * lin_rows + full * full_rows) * H * 2 / cfg["layers"], cfg["layers"]),
        "residual_project": ((lin * H * d["value_size"] + full * H * d["query_size"]) * 2 / cfg["layers"]
                             + (0 if cfg["moe"] else H * cfg["intermediate"] * 2) / 2,
                             cfg["layers"] * (1 if cfg["moe"] else 2)),
        "logits_argmax": (V * H * 2, 1),
        "attention": ((context + 1) * 2 * d["kvs"] * 2, full),
        "delta": (2 * d["recurrent"] * 2, lin),
    }
    # the persistent step is one launch per token: its algorithmic bytes are
    # the whole token's (weights touched + KV read + state read/write)
    out["decode_step"] = (cq35.bytes_per_token(cfg, context)["total"], 1)
    if cfg["moe"]:
        K, I, SI, E = cfg["top_k"], cfg["intermediate"], cfg["shared_intermediate"], cfg["experts"]
        out["moe_gate_up"] = ((K * I + SI) * H * 2 * 2, cfg["layers"])
        out["moe_down"] = ((K * I + SI) * H * 2, cfg["layers"])
        out["moe_router"] = ((E + 1) * H * 4, cfg["layers"])
    else:
        out["swiglu"] = (2 * cfg["intermediate"] * H * 2, cfg["layers"])
    return out


def measured_traffic(config: str) -> dict:
    """HBM bytes per dispatch by kernel class from the committed counter
    summary (two rocprofv3 --pmc passes, FETCH_SIZE then WRITE_SIZE, scaled
    by a copy of known size); empty when none exists for this config."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{config.replace('qwen36-', '').replace('-', '_')}.md")
    try:
        text = open(path).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(block)
    except (OSError, IndexError, ValueError):
        return {}


def measure_kernels(session, tokens, classes, steps_each):
    """Average launch duration of each kernel class from HIP events on the
    session stream (graph replay suspended while timing)."""
    import cq35
    names = cq35.kernel_classes()
    res = {}
    i = 0
    for name in classes:
        kc = names.index(name)
        if name != "decode_step" and session.persistent:
            session.set_persistent(False)  # per-kernel classes exist only on that path
        session.time_kernel(kc)
        for _ in range(steps_each):
            session.decode_next_token(tokens[i])
            i += 1
        ms, n = session.kernel_time()
        res[name] = (ms, n)
        session.time_kernel(-1)
    return res, i


def host_info() -> dict:
    """The host the CPU leg ran on: logical CPUs and the processor model."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(nproc=os.cpu_count(), cpu_model=model,
                omp_num_threads=os.environ.get("OMP_NUM_THREADS"))


def cpu_baseline(cfg, seed, prompt_len, max_steps, budget_s, gpu_model, threads):
    import numpy as np

    import oracle
    oracle.build()
    oracle.lib().ox_set_threads(threads)
    t0 = time.time()
    weights = oracle.synthetic_weights(cfg, seed)
    gen_s = time.time() - t0
    log(f"  CPU weights generated in {gen_s:.1f}s")
    model = oracle.Model(cfg, weights)
    toks = synthetic_tokens(prompt_len + max_steps + 1, cfg["vocab"])
    cs = model.session(prompt_len + max_steps + 1)
    gs = gpu_model.session(prompt_len + max_steps + 1)
    # the prompt as one call: the batched prefill at key_dim 128 on both sides
    ct, cl = cs.step(toks[:prompt_len], 0)
    gl, gt = gs.step_raw(toks[:prompt_len])
    equal_tokens = ct == gt
    equal_logits = bool(np.array_equal(cl, gl))
    steps = 0
    elapsed = 0.0
    pos = prompt_len
    while steps < max_steps and elapsed < budget_s:
        t1 = time.time()
        ct, cl = cs.step([ct], pos)
        elapsed += time.time() - t1
        gl, gt = gs.step_raw([gt])
        equal_tokens &= ct == gt
        equal_logits &= bool(np.array_equal(cl, gl))
        pos += 1
        steps += 1
        log(f"  CPU decode step {steps}: {elapsed:.1f}s so far, tokens equal {equal_tokens}")
    return dict(tokens_per_s=steps / elapsed if elapsed else 0.0, steps=steps, seconds=elapsed,
                weight_gen_s=gen_s, prompt=prompt_len, tokens_equal=bool(equal_tokens),
                logits_equal=equal_logits)


def seeded_state(cfg: dict, capacity: int, position: int, seed: int):
    """BF16 session state of the long-context configuration: key and value
    rows of positions < `position` ~ N(0,1) x 0.1, conv history ~ N(0,1) x 0.1
    and DeltaNet recurrent state ~ N(0,1), seeded; generated with torch's
    generator on the GPU (the same HIP runtime the library uses; the host
    generator takes seconds per 32K-position state) and copied to the host.
    Layout (src/spec.rs:321-362): [layer][key|value][capacity][kv_heads*head_dim],
    then per layer [conv history | recurrent state]."""
    import numpy as np
    import torch
    dev = "cuda" if torch.cuda.is_available() else "cpu"
    kvs = cfg["kv_heads"] * cfg["head_dim"]
    ks, vs = cfg["key_heads"] * cfg["key_dim"], cfg["value_heads"] * cfg["value_dim"]
    conv = 3 * (2 * ks + vs)
    lin = conv + vs * cfg["key_dim"]
    kv = capacity * cfg["layers"] * 2 * kvs
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    out = torch.zeros(kv + cfg["layers"] * lin, dtype=torch.bfloat16, device=dev)
    rows = out[:kv].view(cfg["layers"] * 2, capacity, kvs)
    for r in range(cfg["layers"] * 2):
        rows[r, :position] = (torch.randn(position, kvs, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    tail = out[kv:].view(cfg["layers"], lin)
    tail[:, :conv] = (torch.randn(cfg["layers"], conv, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    tail[:, conv:] = torch.randn(cfg["layers"], lin - conv, generator=g, device=dev).to(torch.bfloat16)
    host = out.view(torch.int16).cpu().numpy().view(np.uint16)
    del out, rows, tail
    if dev == "cuda":
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return host


def long_context_decode(model, cfg: dict, context: int, steps: int, seed: int) -> dict:
    """Batch-1 greedy decode from a seeded state holding `context` cached
    positions (the long-context configuration's per-session work)."""
    import cq35
    warm = 2
    exact_steps = max(2, steps // 4)
    capacity = context + warm + steps + 1 + exact_steps
    t0 = time.time()
    state = seeded_state(cfg, capacity, context, seed + 101)
    s = model.session(capacity)
    s.import_state(0, state)
    s.position = context
    del state
    log(f"long context: {context}-position state generated and imported in {time.time() - t0:.1f}s")
    nxt = 1
    for _ in range(warm):
        nxt = s.decode_next_token(nxt)
    device_sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        nxt = s.decode_next_token(nxt)
    device_sync()
    elapsed = time.perf_counter() - t0
    ms = elapsed / steps * 1e3
    bpt = cq35.bytes_per_token(cfg, context + warm + steps // 2)
    gbs = bpt["total"] / (ms / 1e3) / 1e9
    log(f"long context {context}: {steps / elapsed:.1f} tok/s, {ms:.3f} ms/token, {gbs:.0f} GB/s "
        f"of {bpt['total'] / 1e9:.3f} GB/token (split-K above {s.attention_split} keys)")
    # the same session on the exact single chain (split off): the reference's
    # own order, the rate that meets the logit bar at full depth
    split = s.attention_split
    s.set_attention_split(0)
    nxt = s.decode_next_token(nxt)
    device_sync()
    t0 = time.perf_counter()
    for _ in range(exact_steps):
        nxt = s.decode_next_token(nxt)
    device_sync()
    exact_s = time.perf_counter() - t0
    s.set_attention_split(split)
    log(f"long context {context}, exact single chain: {exact_steps / exact_s:.1f} tok/s")
    return dict(context=context, steps=steps, warmup=warm, tokens_per_s=round(steps / elapsed, 2),
                ms_per_token=round(ms, 4), bytes_per_token=bpt["total"], achieved_gbs=round(gbs, 1),
                frac=round(gbs / HBM_PEAK_GBS, 4), split_keys=split,
                exact_chain=dict(steps=exact_steps, tokens_per_s=round(exact_steps / exact_s, 2),
                                 ms_per_token=round(exact_s / exact_steps * 1e3, 4)),
                decode_path="persistent one-launch step" if s.persistent else "per-kernel launch sequence",
                state="seeded: KV N(0,1) x 0.1, conv history N(0,1) x 0.1, DeltaNet state N(0,1)")


def round_bytes(cfg: dict, sessions: int, context: int, distinct: float) -> dict:
    """Algorithmic HBM bytes of one weight-shared batched MoE round:
    `sessions` tokens at about `context` cached positions each, the
    non-expert weights read once, `distinct` routed experts per layer read
    once each, every session's KV and DeltaNet state."""
    import cq35
    one = cq35.bytes_per_token(cfg, context)
    expert = 3 * cfg["intermediate"] * cfg["hidden"] * 2
    routed_one = cfg["layers"] * cfg["top_k"] * expert
    weights = one["weights"] - routed_one + (sessions - 1) * cfg["hidden"] * 2  # one embedding row per token
    routed = cfg["layers"] * distinct * expert
    return dict(weights=weights, routed_experts=routed, kv=sessions * one["kv"], state=sessions * one["state"],
                total=weights + routed + sessions * (one["kv"] + one["state"]))


def concurrent_long(model, cfg: dict, sessions: int, context: int, steps: int, prefill_tokens: int,
                    chunk: int, seed: int) -> dict:
    """The long-context serving configuration: `sessions` concurrent sessions,
    each holding `context` cached positions (a seeded state: KV N(0,1) x 0.1,
    DeltaNet state N(0,1); one generated state imported into every session,
    each session then decoding from its own first token), `steps` greedy
    decode rounds through cq35_step_batch, and one `prefill_tokens`-token
    prompt on another session, appended in `chunk`-token calls on the matrix
    cores (MFMA projections, experts and attention), one call after each
    decode round until it is done. Aggregate decode tok/s over the whole
    interleaved run."""
    import numpy as np

    import cq35
    capacity = context + steps + 8
    t0 = time.time()
    state = seeded_state(cfg, capacity, context, seed + 202)
    group = []
    for b in range(sessions):
        s = model.session(capacity)
        s.import_state(0, state)
        s.position = context
        group.append(s)
    del state
    log(f"concurrent long context: {sessions} sessions of {context} positions ready in {time.time() - t0:.1f}s")
    pre = model.session(prefill_tokens + 8)
    pre.set_matrix_prefill(pre.MATRIX_PROJECTIONS | pre.MATRIX_EXPERTS | pre.MATRIX_ATTENTION)
    prompt = synthetic_tokens(prefill_tokens + 1, cfg["vocab"])[1:]
    warm = model.session(chunk + 1)  # the chunk kernels' first launch, outside the timing
    warm.set_matrix_prefill(warm.MATRIX_PROJECTIONS | warm.MATRIX_EXPERTS | warm.MATRIX_ATTENTION)
    warm.append_next_token(prompt[:chunk])
    del warm
    nxt = [1000 + 17 * b for b in range(sessions)]
    nxt = cq35.decode_batch(group, nxt)  # one untimed round
    done, decode_s, prefill_s = 0, 0.0, 0.0
    device_sync()
    t0 = time.perf_counter()
    for r in range(steps):
        t1 = time.perf_counter()
        nxt = cq35.decode_batch(group, nxt)
        t2 = time.perf_counter()
        decode_s += t2 - t1
        if done < prefill_tokens:
            n = min(chunk, prefill_tokens - done)
            pre.append_next_token(prompt[done:done + n])
            done += n
            prefill_s += time.perf_counter() - t2
    device_sync()
    wall = time.perf_counter() - t0
    agg = sessions * steps / wall
    log(f"{sessions} sessions x {context} positions, {steps} rounds with a {prefill_tokens}-token chunked "
        f"prefill interleaved: {agg:.1f} decode tok/s aggregate ({wall:.2f}s; decode {decode_s:.2f}s, "
        f"prefill {prefill_s:.2f}s = {prefill_tokens / prefill_s:.0f} tok/s)")
    # distinct routed experts per layer and round, from a few more rounds
    # (outside the timing: the ids are read back per session)
    distinct = []
    for _ in range(4):
        nxt = cq35.decode_batch(group, nxt)
        ids = np.stack([s.router_ids() for s in group])  # [sessions][layers][top_k]
        distinct += [len(np.unique(ids[:, layer, :])) for layer in range(ids.shape[1])]
    rb = round_bytes(cfg, sessions, context + steps // 2, float(np.mean(distinct)))
    round_s = decode_s / steps
    log(f"  per round: {rb['total'] / 1e9:.2f} GB ({np.mean(distinct):.1f} distinct experts per layer), "
        f"{round_s * 1e3:.2f} ms, {rb['total'] / round_s / 1e9:.0f} GB/s")
    return dict(sessions=sessions, context=context, steps=steps, wall_s=round(wall, 3),
                decode_tokens_per_s=round(agg, 1), decode_only_tokens_per_s=round(sessions * steps / decode_s, 1),
                ms_per_round=round(round_s * 1e3, 3), bytes_per_round=int(rb["total"]),
                bytes_per_round_parts={k: int(v) for k, v in rb.items() if k != "total"},
                distinct_experts_per_layer=round(float(np.mean(distinct)), 2),
                achieved_gbs=round(rb["total"] / round_s / 1e9, 1),
                decode_step_roofline_frac=round(rb["total"] / round_s / 1e9 / HBM_PEAK_GBS, 4),
                prefill=dict(tokens=prefill_tokens, chunk=chunk, seconds=round(prefill_s, 3),
                             tokens_per_s=round(prefill_tokens / prefill_s, 1),
                             path="matrix-core prefill (MFMA projections, experts and attention), one call per round"),
                state="seeded: KV N(0,1) x 0.1, conv history N(0,1) x 0.1, DeltaNet state N(0,1); one state "
                      "imported into every session",
                split_keys=group[0].attention_split,
                decode_path="cq35_step_batch: weight-shared MoE step (projections, router, shared expert and head "
                            "read once per round, each distinct routed expert once; per-session split-K "
                            "attention)")


def batch_sessions(config: str, sessions: int, context: int, steps: int, seed: int) -> dict:
    """The batch-16 configuration: `sessions` independent sessions of
    `config`, each prefilled with its own `context`-token prompt, then
    `steps` greedy decode rounds through cq35_step_batch, against one session
    decoding alone over the same rounds."""
    import cq35
    cfg = cq35.preset(config)
    model = cq35.Model.synthetic(cfg, seed=seed)
    capacity = context + 2 * steps + 16  # exact rounds, then as many matrix-core rounds
    tokens = synthetic_tokens(sessions * context + 1, cfg["vocab"])
    group, nxt = [], []
    for b in range(sessions):
        s = model.session(capacity)
        nxt.append(s.append_next_token(tokens[b * context:(b + 1) * context]))
        group.append(s)
    for _ in range(2):
        nxt = cq35.decode_batch(group, nxt)
    device_sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        nxt = cq35.decode_batch(group, nxt)
    device_sync()
    batched = time.perf_counter() - t0
    # the same sessions with the products on MFMA (matrix-core decode
    # selected on every session: tolerance-level, tests/test_gpu_batch_matrix.py)
    for s in group:
        s.set_matrix_decode(True)
    mx_steps = steps
    for _ in range(2):
        nxt = cq35.decode_batch(group, nxt)
    device_sync()
    t0 = time.perf_counter()
    for _ in range(mx_steps):
        nxt = cq35.decode_batch(group, nxt)
    device_sync()
    matrix = time.perf_counter() - t0
    one = model.session(capacity)
    x = one.append_next_token(tokens[:context])
    for _ in range(2):
        x = one.decode_next_token(x)
    device_sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        x = one.decode_next_token(x)
    device_sync()
    alone = time.perf_counter() - t0
    log(f"{sessions} {config} sessions: {sessions * steps / batched:.1f} tok/s aggregate "
        f"({batched / steps * 1e3:.3f} ms per round); one session {steps / alone:.1f} tok/s")
    if mx_steps:
        log(f"{sessions} {config} sessions, matrix-core products: {sessions * mx_steps / matrix:.1f} tok/s "
            f"aggregate ({matrix / mx_steps * 1e3:.3f} ms per round)")
    return dict(config=config, sessions=sessions, context=context, steps=steps,
                tokens_per_s=round(sessions * steps / batched, 1), ms_per_round=round(batched / steps * 1e3, 4),
                single_session_tokens_per_s=round(steps / alone, 1),
                path=("cq35_step_batch: weight-shared decode step (each layer's weights read once for all "
                      "sessions' tokens, per-token arithmetic bit-identical to a session stepped alone)"),
                matrix_core=dict(steps=mx_steps,
                                 tokens_per_s=round(sessions * mx_steps / matrix, 1) if mx_steps else None,
                                 ms_per_round=round(matrix / mx_steps * 1e3, 4) if mx_steps else None,
                                 path="the same step with its products on MFMA (tolerance-level)"))


def dense_decode(config: str, context: int, steps: int, seed: int) -> dict:
    """Batch-1 greedy decode of a dense configuration (the 0.8B and 2B
    shapes): a `context`-token prompt in one call, two warm-up steps, then
    `steps` timed decode steps; the roofline fraction is the algorithmic
    bytes per token at the mean context over the step time."""
    import cq35
    cfg = cq35.preset(config)
    model = cq35.Model.synthetic(cfg, seed=seed)
    s = model.session(context + steps + 8)
    x = s.append_next_token(synthetic_tokens(context, cfg["vocab"]))
    for _ in range(2):
        x = s.decode_next_token(x)
    device_sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        x = s.decode_next_token(x)
    device_sync()
    dt = time.perf_counter() - t0
    bpt = cq35.bytes_per_token(cfg, context + 2 + steps // 2)["total"]
    gbs = bpt * steps / dt / 1e9
    log(f"dense {config}: {steps / dt:.1f} tok/s batch 1 ({dt / steps * 1e3:.3f} ms/token, "
        f"{gbs:.0f} GB/s of {bpt / 1e9:.3f} GB/token)")
    return dict(config=config, context=context, steps=steps, tokens_per_s=round(steps / dt, 1),
                ms_per_token=round(dt / steps * 1e3, 4), bytes_per_token=bpt, achieved_gbs=round(gbs, 1),
                frac=round(gbs / HBM_PEAK_GBS, 4),
                decode_path="persistent one-launch step" if s.persistent else "per-kernel launch sequence")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--runs", type=int, default=3, help="timed runs (fresh session each); mean and stddev")
    ap.add_argument("--config", default="qwen36-35b-a3b")
    ap.add_argument("--context", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-kernel-timing", action="store_true")
    ap.add_argument("--per-kernel-timing", action="store_true",
                    help="also time each kernel class of the per-kernel launch sequence")
    ap.add_argument("--per-kernel", action="store_true",
                    help="decode through the per-kernel launch sequence instead of the persistent step")
    # the box's CPU share for one GPU is 16 cores (OMP_NUM_THREADS there), so
    # the restatement uses that many threads, not every core the host shows
    ap.add_argument("--cpu-threads", type=int,
                    default=min(int(os.environ.get("OMP_NUM_THREADS", "16") or 16), os.cpu_count() or 1))
    ap.add_argument("--cpu-steps", type=int, default=32)
    ap.add_argument("--cpu-budget", type=float, default=25.0)
    ap.add_argument("--prompt-per-token", action="store_true",
                    help="append the prompt one token per call instead of one batched call")
    ap.add_argument("--no-matrix-prefill", action="store_true",
                    help="skip the matrix-core prefill measurement")
    ap.add_argument("--long-context", type=int, default=32768,
                    help="cached positions of the long-context decode leg (0 skips it)")
    ap.add_argument("--long-steps", type=int, default=128)
    ap.add_argument("--concurrent", type=int, default=8,
                    help="sessions of the concurrent long-context leg (0 skips it)")
    ap.add_argument("--concurrent-steps", type=int, default=128)
    ap.add_argument("--concurrent-prefill", type=int, default=4096)
    # the reference's server prefills prompts in absolute 1024-token blocks
    # (PREFILL_BLOCK, src/server/prefix_cache.rs:4; engine.rs:330)
    ap.add_argument("--concurrent-chunk", type=int, default=1024,
                    help="tokens per interleaved prefill call of the concurrent leg")
    ap.add_argument("--batch-sessions", type=int, default=16,
                    help="sessions of the batch-16 leg (0 skips it)")
    ap.add_argument("--batch-config", default="qwen35-2b")
    ap.add_argument("--batch-steps", type=int, default=64)
    ap.add_argument("--dense", default="qwen35-0.8b:512,qwen35-2b:1024",
                    help="dense batch-1 decode legs, config:context pairs ('' for none)")
    ap.add_argument("--dense-steps", type=int, default=256)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run one device copy of this size (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "The token loop would shard by placing whole sessions per GPU, with no communication.",
              file=sys.stderr)
        return 2

    import cq35
    cfg = cq35.preset(args.config)
    if args.copy_probe:
        copy_probe(args.copy_probe)
    ceiling = copy_ceiling()
    t0 = time.time()
    model = cq35.Model.synthetic(cfg, seed=args.seed)
    log(f"weights: {model.weight_bytes() / 1e9:.2f} GB generated on device in {time.time() - t0:.1f}s")
    per_kernel_classes = (
        ["project", "moe_gate_up", "moe_down", "residual_project", "logits_argmax", "attention",
         "delta", "moe_router"] if cfg["moe"] else
        ["project", "swiglu", "residual_project", "logits_argmax", "attention", "delta"])
    timing_steps = 3
    capacity = args.context + args.warmup + args.steps + (len(per_kernel_classes) + 1) * timing_steps + 1
    tokens = synthetic_tokens(capacity, cfg["vocab"])
    session = model.session(capacity)
    if args.per_kernel and session.persistent:
        session.set_persistent(False)
    persistent = session.persistent
    if args.no_kernel_timing:
        timing_classes = []
    elif persistent:
        timing_classes = ["decode_step"] + (per_kernel_classes if args.per_kernel_timing else [])
    else:
        timing_classes = per_kernel_classes
    batched_prompt = not args.prompt_per_token and cfg["key_dim"] == 128 and args.context >= 2
    device_sync()
    t0 = time.perf_counter()
    if batched_prompt:
        # one call, as the reference's benchmark prefills its context
        # (main.rs:393-445 -> prefill_next_token -> text-batch)
        session.append_next_token(tokens[:args.context])
    else:
        for t in tokens[:args.context]:
            session.append_next_token([t])
    device_sync()
    prefill_s = time.perf_counter() - t0
    prefill = dict(tokens=args.context, seconds=round(prefill_s, 4),
                   tokens_per_s=round(args.context / prefill_s, 1) if prefill_s > 0 else None,
                   path="batched prefill, one call" if batched_prompt else "one token per call")
    log(f"prompt of {args.context} tokens ({prefill['path']}) in {prefill_s:.3f}s")
    if batched_prompt and not args.no_matrix_prefill:
        # the same prompt on a second session with the matrix-core components
        # (MFMA accumulation order; the decode below runs on the exact session)
        ms_ = model.session(args.context + 1)
        ms_.set_matrix_prefill(ms_.MATRIX_PROJECTIONS | ms_.MATRIX_EXPERTS | ms_.MATRIX_ATTENTION)
        ms_.append_next_token(tokens[:args.context])  # warm the kernels
        ms_ = model.session(args.context + 1)
        ms_.set_matrix_prefill(ms_.MATRIX_PROJECTIONS | ms_.MATRIX_EXPERTS | ms_.MATRIX_ATTENTION)
        device_sync()
        t0 = time.perf_counter()
        ms_.append_next_token(tokens[:args.context])
        device_sync()
        mp_s = time.perf_counter() - t0
        del ms_
        prefill["matrix_core"] = dict(seconds=round(mp_s, 4), tokens_per_s=round(args.context / mp_s, 1),
                                      components="projections+experts+attention (MFMA accumulation order)")
        log(f"prompt of {args.context} tokens, matrix-core prefill: {mp_s:.3f}s")
    # `runs` timed runs (the reference's --bench-runs, main.rs:459-471): each
    # a fresh session with the prompt, W untimed then K timed greedy steps;
    # the reported rate is their mean, with the standard deviation
    rates = []
    for run in range(args.runs):
        if run > 0:
            session = model.session(capacity)
            if args.per_kernel and session.persistent:
                session.set_persistent(False)
            if batched_prompt:
                session.append_next_token(tokens[:args.context])
            else:
                for t in tokens[:args.context]:
                    session.append_next_token([t])
        base = args.context
        nxt = tokens[base]
        for _ in range(args.warmup):
            nxt = session.decode_next_token(nxt)
        base += args.warmup
        device_sync()
        t0 = time.perf_counter()
        for _ in range(args.steps):  # greedy: each step feeds back the previous token
            nxt = session.decode_next_token(nxt)
        device_sync()
        elapsed = time.perf_counter() - t0
        base += args.steps
        rates.append(args.steps / elapsed)
        log(f"decode run {run + 1}: {rates[-1]:.1f} tok/s")
    value = sum(rates) / len(rates)
    stddev = (sum((r - value) ** 2 for r in rates) / (len(rates) - 1)) ** 0.5 if len(rates) > 1 else 0.0
    ms = 1e3 / value
    ctx_avg = args.context + args.warmup + args.steps // 2
    bpt = cq35.bytes_per_token(cfg, ctx_avg)
    step_gbs = bpt["total"] / (ms / 1e3) / 1e9
    log(f"decode: {value:.1f} +- {stddev:.1f} tok/s over {len(rates)} runs, {ms:.3f} ms/token, "
        f"{step_gbs:.0f} GB/s of {bpt['total'] / 1e9:.3f} GB/token")

    roofline = None
    kernels = {}
    if timing_classes:
        kb = kernel_bytes(cfg, ctx_avg)
        res, used = measure_kernels(session, tokens[base:], timing_classes, timing_steps)
        base += used
        for name, (kms, n) in res.items():
            if n == 0:
                continue
            per_launch = kms / n
            by = kb.get(name, (None, None))[0]
            kernels[name] = dict(ms_per_step=kms / timing_steps, avg_launch_us=per_launch * 1e3,
                                 launches_per_step=n / timing_steps,
                                 gbs=(by / (per_launch / 1e3) / 1e9) if by else None)
        dom = "decode_step" if "decode_step" in kernels else max(kernels, key=lambda k: kernels[k]["ms_per_step"])
        by, _ = kb[dom]
        avg_s = kernels[dom]["avg_launch_us"] / 1e6
        achieved = by / avg_s / 1e9
        tr = measured_traffic(args.config).get(dom)
        traffic = tr["fetch_bytes"] + tr["write_bytes"] if tr else None
        roofline = dict(kernel=dom, bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS,
                        unit="GB/s", frac=round(achieved / HBM_PEAK_GBS, 4), traffic=traffic,
                        bytes_per_launch=int(by), avg_launch_us=round(kernels[dom]["avg_launch_us"], 2),
                        copy_ceiling_gbs=ceiling["gbs"], frac_of_copy_ceiling=round(achieved / ceiling["gbs"], 4))
        for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["ms_per_step"]):
            log(f"  {k:18s} {v['ms_per_step']:.3f} ms/step  {v['avg_launch_us']:.1f} us/launch"
                + (f"  {v['gbs']:.0f} GB/s" if v["gbs"] else ""))

    long_ctx = None
    if args.long_context > 0:
        del session
        long_ctx = long_context_decode(model, cfg, args.long_context, args.long_steps, args.seed)
    concurrent = None
    if args.concurrent > 0 and args.long_context > 0:
        concurrent = concurrent_long(model, cfg, args.concurrent, args.long_context, args.concurrent_steps,
                                     args.concurrent_prefill, args.concurrent_chunk, args.seed)
    batch = None
    if args.batch_sessions > 0:
        batch = batch_sessions(args.batch_config, args.batch_sessions, 1024, args.batch_steps, args.seed)

    dense = []
    for item in filter(None, args.dense.split(",")):
        name, ctx = item.split(":")
        dense.append(dense_decode(name, int(ctx), args.dense_steps, args.seed))

    cpu = None
    if not args.no_cpu:
        need = model.weight_bytes()
        try:
            import psutil
            avail = psutil.virtual_memory().available
        except Exception:
            avail = need * 4
        if avail > need * 1.3:
            log(f"CPU baseline: restatement on {args.cpu_threads} threads ...")
            c = cpu_baseline(cfg, args.seed, 4, args.cpu_steps, args.cpu_budget, model, args.cpu_threads)
            cpu = dict(value=round(c["tokens_per_s"], 4), unit="tokens/s", cores=args.cpu_threads,
                       kind="port", host=host_info(),
                       sample=(f"{args.config} shape, same synthetic weights; 4-token prompt (one call) then "
                               f"{c['steps']} timed batch-1 decode steps ({c['seconds']:.1f}s; weight "
                               f"generation {c['weight_gen_s']:.1f}s not timed). The prompt is 4 tokens, not "
                               f"{args.context}: the restatement's exact-order prefill costs about as much per "
                               "token as a decode step (0.4 s at 35B), so the configured prompt alone would "
                               "take minutes; the decode steps are what is timed"),
                       gpu_parity=dict(greedy_tokens_equal=c["tokens_equal"],
                                       bf16_logits_equal=c["logits_equal"], steps=c["steps"] + 4))
            log(f"CPU: {c['tokens_per_s']:.3f} tok/s; GPU/CPU greedy equal={c['tokens_equal']} "
                f"logits equal={c['logits_equal']}")
        else:
            log(f"CPU baseline skipped: {avail / 1e9:.0f} GB host memory available, need {need / 1e9:.0f} GB")

    line = dict(
        metric="decode tokens/sec at batch 1 (35B-A3B-shape MoE) + % of HBM roofline",
        value=round(value, 3), unit="tokens/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
        runs=dict(count=len(rates), mean=round(value, 3), stddev=round(stddev, 3),
                  values=[round(r, 2) for r in rates]),
        ms_per_step=round(ms, 4), higher_is_better=True, scaling="weak", vs_baseline=None,
        dtype="bf16", data="synthetic (seeded random-init weights, LCG prompt ids)",
        config=dict(workload=f"{args.config} batch-1 greedy decode", model=args.config,
                    global_batch=1, seq_len=args.context, context_avg=ctx_avg, parallelism="none",
                    decode_path="persistent one-launch step" if persistent else "per-kernel launch sequence"),
        step_roofline=dict(bytes_per_token=bpt["total"], achieved_gbs=round(step_gbs, 1),
                           frac=round(step_gbs / HBM_PEAK_GBS, 4),
                           frac_of_copy_ceiling=round(step_gbs / ceiling["gbs"], 4)),
        copy_ceiling=ceiling,
        roofline=roofline, kernels=kernels, cpu_baseline=cpu,
        prefill=prefill, long_context=long_ctx, concurrent_long_context=concurrent, batch_sessions=batch,
        dense_decode=dense or None,
    )
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
