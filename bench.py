#!/usr/bin/env python3
"""Benchmark of the KV-cache self-speculative decode path on one MI355X.

Workload (default): random-init Pulsar-283M in bf16 (weights N(0, 0.02), reference constant
init elsewhere), batch 16, 2048-token uniform-random prompts, sampled self-speculative decode
with temperature 0.8, top-p 0.95, repetition penalty 1.15 (the reference default), 256 new
tokens per sequence, draft length 4, stop ids disabled so every sequence produces exactly
256 tokens. Draft length 4 is the draft-block schedule: up to 4 pulse-0 drafts per round, one
all-pulse verify of the block, drafts accepted down the block by the reference's equal-draw
rule. The reference's own schedule (draft length 1, src/infer.py:623-731) is timed beside it
(`exact_schedule`); `--draft-len 0` makes it the headline.

A step = one generation of the whole batch from the prefilled KV cache: rewind (redraw the
first token from the saved prefill logits with a new seed) and decode until every sequence
has its 256 tokens. Prefill runs once, untimed, and is reported separately.

Prints one JSON line: value = accepted tokens/s over the K timed steps; roofline = the
dominant kernel class measured with HIP events (eager profiled generation), against its
algorithmic bytes; cpu_baseline = the oracle (PyTorch CPU restatement of the reference path)
decoding one sequence of the same workload on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "pulsar-300m_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "accepted tokens/s at 1 GPU (batch 16, ctx 2k); % HBM roofline; acceptance rate"
HBM_PEAK = 8.0e12
MFMA_BF16_PEAK = 2.5e15  # dense bf16 matrix-core peak (no sparsity)
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_c2_b16_t2048.md")
BLOCK_TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_c2_draft4_b16_t2048.md")
# kernel classes by the short names of their templates (gemm EPI: 0 store, 1 qkv + gate,
# 2 residual add, 3 SwiGLU, 4 logits), for class averages over every template of a class
CLASS_PREFIXES = {
    "attention": ("attn_decode_unit_kernel<",),
    "routed_gate_up": ("gemm_bf16_kernel<3,", "gemm_bf16_lds_kernel<3,", "gemm_bf16_mid_kernel<3,"),
    "routed_down": ("gemm_bf16_kernel<0,", "gemm_bf16_lds_kernel<0,", "gemm_bf16_mid_kernel<0,"),
    "qkv_gate_gemm": ("gemm_bf16_kernel<1,", "gemm_bf16_lds_kernel<1,", "gemm_bf16_mid_kernel<1,"),
    "wo_gemm": ("gemm_bf16_kernel<2,", "gemm_bf16_lds_kernel<2,", "gemm_bf16_mid_kernel<2,"),
    "lm_head": ("gemm_bf16_kernel<4,", "gemm_bf16_lds_kernel<4,"),
    "router": ("norm_router_kernel<",),
    "moe_combine": ("moe_combine_rows_kernel<",),
    "sample": ("sample_kernel<",),
    "pulse_input": ("pulse_input_kernel<",),
    "pulse_output": ("pulse_output_kernel<",),
    "controller": ("controller_kernel", "controller_block_kernel"),
}
VERIFY_TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_verify_b64_ctx8192.md")


def _short_kernel(name: str) -> str:
    import re
    name = name.replace("(anonymous namespace)::", "").replace("pulsar::", "")
    return re.sub(r"\(.*", "", name).replace("void ", "").strip()


def _phase_rows(rows: list, phase: str) -> list:
    """Dispatches of one phase of a bench run. The last prefill is the run of dispatches
    from just after the controller launch that precedes its last prefill kernel up to the
    controller launch that ends it (drawing the first tokens); decode is everything after."""
    names = [r["Kernel_Name"] for r in rows]
    ctl = [i for i, n in enumerate(names) if "controller_kernel" in n or "controller_block" in n]
    pre = [i for i, n in enumerate(names) if "prefill" in n]
    if not pre:
        end = ctl[0] if ctl else -1
        return rows[end + 1:] if phase == "decode" else []
    last = pre[-1]
    end = next((i for i in ctl if i > last), len(rows))
    start = max((i for i in ctl if i < last), default=-1) + 1
    return rows[end + 1:] if phase == "decode" else rows[start:end]


def _csv(directory: str, suffix: str) -> list:
    import csv
    import glob
    paths = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not paths:
        raise SystemExit(f"no *{suffix} under {directory}")
    with open(paths[0]) as f:
        return list(csv.DictReader(f))


def _busy_launches(v: list) -> list:
    """The launches of a kernel that did work: kernels whose row set can be empty (the output
    head and the sampler on steps without logits rows, exact schedule) exit at once there.
    When a kernel's durations split into such a cluster under 4 us and one at least 3 times
    longer (10th against 90th percentile), the launches above the geometric mean of the two
    percentiles; otherwise all of them."""
    s = sorted(v)
    if len(s) < 8:
        return v
    lo, hi = s[len(s) // 10], s[(9 * len(s)) // 10]
    if hi < 3 * lo or lo > 4000:
        return v
    cut = (lo * hi) ** 0.5
    return [x for x in v if x >= cut]


def rocprof_summary(directory: str, phase: str = "decode") -> str:
    """Markdown table of one phase's kernel durations from a rocprofv3 kernel trace (csv):
    all dispatches, and the dispatches that did work (`_busy_launches`)."""
    from collections import defaultdict
    rows = _phase_rows(_csv(directory, "kernel_trace.csv"), phase)
    agg = defaultdict(list)
    for r in rows:
        agg[_short_kernel(r["Kernel_Name"])].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    total = sum(sum(v) for v in agg.values())
    out = ["| kernel | dispatches | avg us | total ms | share | busy dispatches | busy avg us |",
           "|---|---|---|---|---|---|---|"]
    for k, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        b = _busy_launches(v)
        out.append(f"| `{k}` | {len(v)} | {sum(v) / len(v) / 1e3:.2f} | {sum(v) / 1e6:.2f} | "
                   f"{100 * sum(v) / total:.1f}% | {len(b)} | {sum(b) / len(b) / 1e3:.2f} |")
    out.append(f"\n{phase.capitalize()} kernel time {total / 1e6:.2f} ms over {len(rows)} dispatches.")
    return "\n".join(out)


def pmc_summary(fetch_dir: str, write_dir: str, fetch_copy: str, write_copy: str,
                copy_mib: int) -> str:
    """Calibrated HBM bytes per decode dispatch from FETCH_SIZE / WRITE_SIZE runs."""
    from collections import defaultdict
    res = {}
    lines = []
    for ctr, d, dc in (("FETCH_SIZE", fetch_dir, fetch_copy), ("WRITE_SIZE", write_dir, write_copy)):
        cal = [float(r["Counter_Value"]) for r in _csv(dc, "counter_collection.csv")
               if "copyBuffer" in r["Kernel_Name"] and float(r["Counter_Value"]) > copy_mib * 256]
        factor = copy_mib * 1024 / (sum(cal) / len(cal))
        lines.append(f"- {ctr}: a {copy_mib} MiB device-to-device copy counts "
                     f"{sum(cal) / len(cal):.1f} KiB per dispatch -> scale factor {factor:.4f}")
        agg = defaultdict(list)
        for r in _phase_rows(_csv(d, "counter_collection.csv"), "decode"):
            agg[_short_kernel(r["Kernel_Name"])].append(float(r["Counter_Value"]))
        for k, v in agg.items():
            res.setdefault(k, {})[ctr] = round(sum(v) / len(v) * factor * 1024)
        # class averages over every dispatch of the class's templates ("class:<name>")
        for cls, pre in CLASS_PREFIXES.items():
            v = [x for k, vals in agg.items() if k.startswith(pre) for x in vals]
            if v:
                res.setdefault("class:" + cls, {})[ctr] = round(sum(v) / len(v) * factor * 1024)
    out = lines + ["", "| kernel | fetch MB / dispatch | write MB / dispatch |", "|---|---|---|"]
    for k, v in sorted(res.items(), key=lambda kv: -kv[1].get("FETCH_SIZE", 0)):
        if k.startswith("class:"):
            continue
        out.append(f"| `{k}` | {v.get('FETCH_SIZE', 0) / 1e6:.3f} | {v.get('WRITE_SIZE', 0) / 1e6:.3f} |")
    out += ["", "Class averages over every dispatch of the class's templates:", "",
            "| class | fetch MB / dispatch | write MB / dispatch |", "|---|---|---|"]
    for k, v in sorted(res.items(), key=lambda kv: -kv[1].get("FETCH_SIZE", 0)):
        if k.startswith("class:"):
            out.append(f"| {k[6:]} | {v.get('FETCH_SIZE', 0) / 1e6:.3f} | "
                       f"{v.get('WRITE_SIZE', 0) / 1e6:.3f} |")
    out += ["", "```json", json.dumps(res, sort_keys=True), "```"]
    return "\n".join(out)


def recorded_traffic(kernels: list, path: str = None):
    """HBM bytes per launch of a kernel class from a committed PMC summary (default: the c2
    decode summary), or None."""
    try:
        with open(path or TRAFFIC_PROFILE) as f:
            text = f.read()
        blob = json.loads(text.split("```json", 1)[1].split("```", 1)[0])
    except (OSError, IndexError, ValueError):
        return None
    total = 0
    for k in kernels:
        if k not in blob:
            return None
        total += blob[k].get("FETCH_SIZE", 0) + blob[k].get("WRITE_SIZE", 0)
    return total


DECODE_TRACE_PROFILE = os.path.join(ROOT, "profiles", "decode_kernels_c2_b16_t2048.md")
BLOCK_TRACE_PROFILE = os.path.join(ROOT, "profiles", "decode_kernels_c2_draft4_b16_t2048.md")


def recorded_kernel_us(cls: str, path: str):
    """Average kernel-trace duration (us) of a kernel class from a committed rocprofv3
    summary table (`| kernel | dispatches | avg us | ...`), weighted by dispatches over every
    template of the class (CLASS_PREFIXES), or None."""
    try:
        with open(path) as f:
            lines = f.read().splitlines()
    except OSError:
        return None
    n = tot = 0.0
    for line in lines:
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) < 3 or not cells[0].startswith("`"):
            continue
        name = cells[0].strip("`")
        if not name.startswith(CLASS_PREFIXES.get(cls, (cls,))):
            continue
        try:
            d, us = float(cells[1]), float(cells[2])
        except ValueError:
            continue
        n += d
        tot += d * us
    return tot / n if n else None


def trace_fraction(roof: dict, cls: str, path: str) -> None:
    """Add to a roofline object the class's kernel-trace average from the committed summary
    at `path` and the fraction of the HBM peak that follows from it (the event span also
    holds the command processor's dispatch, so the event-timed `frac` is the lower one)."""
    us = recorded_kernel_us(cls, path)
    roof["kernel_trace_us"] = round(us, 2) if us else None
    roof["frac_kernel_trace"] = (round(roof["bytes_per_launch"] / (us * 1e-6) / HBM_PEAK, 4)
                                 if us else None)
    roof["kernel_trace_profile"] = os.path.relpath(path, ROOT)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def profile_generation(eng, cfg, es, seed):
    """One eagerly profiled generation (HIP events around every kernel class on the engine's
    stream, the device kept busy ahead of each group) with the algorithmic bytes of each
    step's row set."""
    from pulsar_engine import traffic

    eng.rewind(seed)
    eng.profile(True)
    totals = {c: 0.0 for c in traffic.CLASSES}
    steps = 0
    while not eng.state()[:, 0].all() and steps < 4 * (eng.max_new + 2) * 3:
        eng.step(1)
        steps += 1
        rows = [(int(r[0]), int(r[2]), int(r[3])) for r in eng.rows(last=True)]
        n_lrows = int(eng.last_ctl()[1])
        b = traffic.step_bytes(cfg, es, rows, eng.expert_counts(), n_lrows)
        for k, v in b.items():
            totals[k] += v
    prof = eng.profile_read()
    eng.profile(False)
    return prof, totals, steps


def verify_microbench(model, cfg, es, args):
    """Verify-step microbenchmark: batch 64 sequences with a synthetic bf16 cache of 8192
    positions (every K/V element ~ N(0, 1)), one verify of a 5-token block (4 drafts + 1) per
    sequence through every pulse of every layer, graph-replayed. Reports ms per verify, the
    whole verify's algorithmic bytes against the HBM peak, and the attention kernel's
    per-launch bytes against its event-timed launch duration (eager profiled verify)."""
    import numpy as np
    import torch

    from pulsar_engine import traffic
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    B, ctx, n = args.verify_batch, args.verify_ctx, args.verify_tokens
    blocks = np.stack([W.uniform_ids(7, f"verify_block_{b}", n, cfg.vocab_size) for b in range(B)])
    eng = HipEngine(model, batch=B, max_prompt=1, max_new=8, temperature=0.0, stop_ids=[],
                    draft_len=n - 1, max_ctx=ctx + 16)
    eng.fill_kv(ctx, seed=5)
    eng.verify(blocks, graph=True)
    for _ in range(3):
        eng.verify(None, graph=True)
    torch.cuda.synchronize()
    reps = args.verify_reps
    t0 = time.perf_counter()
    for _ in range(reps):
        eng.verify(None, graph=True)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / reps * 1e3
    counts = eng.expert_counts()  # the last pass's; every expert has rows at 320 rows a pass
    P = cfg.default_pulses
    by_class: dict = {}
    for k in range(P):
        rows = [(b, k, ctx + i) for b in range(B) for i in range(n)]
        step = traffic.step_bytes(cfg, es, rows, counts, B * n if k == P - 1 else 0)
        for c, v in step.items():
            by_class[c] = by_class.get(c, 0.0) + v
    total = sum(by_class.values())
    eng.profile(True)
    eng.verify(None)
    prof = eng.profile_read()
    eng.profile(False)
    att_ms, att_n = prof["attention"]
    att_bytes = by_class["attention"] / max(att_n, 1)
    att_s = att_ms / max(att_n, 1) / 1e3
    # query columns of a unit (4 per row) and 64-key blocks per wave: caches past 16 splits
    # of 256 keys take 4 in sliding-window layers and 8 in global layers, 1 otherwise
    cols = 8 if n <= 2 else 16 if n <= 4 else 32
    lng = (ctx + 16 + 63 + 255) // 256 > 16
    n_loc = sum(1 for i in range(cfg.n_core) if cfg.is_local(i))
    n_glob = cfg.n_core - n_loc
    k_loc = f"attn_decode_unit_kernel<{cols}, {4 if lng else 1}>"
    k_glob = f"attn_decode_unit_kernel<{cols}, {8 if lng else 1}>"
    att_kernels = sorted({k_loc, k_glob})
    t_loc = recorded_traffic([k_loc], VERIFY_TRAFFIC_PROFILE)
    t_glob = recorded_traffic([k_glob], VERIFY_TRAFFIC_PROFILE)
    att_traffic = ((n_loc * t_loc + n_glob * t_glob) / cfg.n_core
                   if t_loc is not None and t_glob is not None else None)
    per_class = {c: {"ms": round(v[0], 3), "launches": v[1],
                     "us_per_launch": round(v[0] / v[1] * 1e3, 2),
                     "GB_per_s": round(by_class.get(c, 0.0) / max(v[0], 1e-9) / 1e6, 1)}
                 for c, v in prof.items() if v[1] and c != "event_pair"}
    # secondary: matrix-core use of the verify's GEMMs (rows of one pass each launch; top-k
    # assignments plus the shared expert over every row), against the dense bf16 peak
    D, R = cfg.d_model, B * n
    gemm_flops = {
        "qkv_gate_gemm": 2.0 * R * D * (cfg.qkv_dim + cfg.n_heads),
        "wo_gemm": 2.0 * R * cfg.q_dim * D,
        "routed_gate_up": 2.0 * D * R * cfg.top_k * 2 * cfg.d_expert,
        "routed_down": 2.0 * D * R * cfg.top_k * cfg.d_expert,
        "shared_gate_up": 2.0 * D * R * 2 * cfg.d_shared,
        "shared_down": 2.0 * D * R * cfg.d_shared,
    }
    for sh, ro in (("shared_gate_up", "routed_gate_up"), ("shared_down", "routed_down")):
        if not prof.get(sh, (0.0, 0))[1]:  # the shared expert rode in the routed launch
            gemm_flops[ro] += gemm_flops.pop(sh)
    gemm_mfma = {}
    for c, fl in gemm_flops.items():
        c_ms, c_n = prof.get(c, (0.0, 0))
        if c_n:
            tf = fl / (c_ms / c_n / 1e3) / 1e12
            gemm_mfma[c] = {"gflop_per_launch": round(fl / 1e9, 3), "TFLOP_per_s": round(tf, 1),
                            "frac": round(tf * 1e12 / MFMA_BF16_PEAK, 4)}
    eng.close()
    return {
        "workload": f"verify of {n} tokens (4 drafts + 1) for each of {B} sequences over a "
                    f"synthetic bf16 cache of {ctx} positions (K/V ~ N(0,1)), every pulse of "
                    f"every layer, graph-replayed",
        "ms_per_verify": round(ms, 4),
        "algorithmic_bytes": int(total),
        "weight_bytes": int(sum(v for c, v in by_class.items() if c != "attention")),
        "kv_bytes": int(by_class["attention"]),
        "hbm_frac": round(total / (ms / 1e3) / HBM_PEAK, 4),
        "roofline": {"bound": "hbm", "kernel": "attention",
                     "kernels": att_kernels,
                     "achieved": round(att_bytes / att_s / 1e9, 1), "peak": 8000.0,
                     "unit": "GB/s", "frac": round(att_bytes / att_s / HBM_PEAK, 4),
                     "bytes_per_launch": int(att_bytes), "avg_launch_us": round(att_s * 1e6, 2),
                     "traffic": round(att_traffic / 1e6, 3) if att_traffic else None,
                     "traffic_unit": "MB per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                     "copy-calibrated, averaged over the layer types by "
                                     "launch count)"},
        "kernel_profile": per_class,
        "gemm_mfma": gemm_mfma,
    }


def run_workload(model, cfg, prompts, n_new, temperature, top_p, rp, steps, warmup, es=2,
                 profile=True, draft_len=0, label="", speculative=True,
                 early_exit_threshold=None, traffic_path=None, keep_seq0=0, trace_path=None):
    """Timed generations of a batch from one prefill: each generation rewinds (redraws the
    first tokens from the saved prefill logits with a new seed) and decodes until every
    sequence has n_new tokens (no stop ids). Returns accepted tokens/s, acceptance, the
    whole generation's algorithmic bytes against the HBM peak and, from one eagerly
    profiled generation, the dominant kernel class's bytes per launch against its
    event-timed launch duration. keep_seq0 > 0 also returns the first keep_seq0 tokens of
    sequence 0 in the last timed generation and their kinds (1: an accepted draft)."""
    import numpy as np
    import torch

    from pulsar_engine.engine import HipEngine

    B, T = prompts.shape
    eng = HipEngine(model, batch=B, max_prompt=T, max_new=n_new, temperature=temperature,
                    top_p=top_p, repetition_penalty=rp, stop_ids=[], seed=1, draft_len=draft_len,
                    speculative=speculative, early_exit_threshold=early_exit_threshold)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.prefill(prompts)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    exits = np.zeros(cfg.default_pulses, np.int64)

    def generation(seed):
        eng.rewind(seed)
        n = eng.run(check_every=16)
        st = eng.state()
        return n, int(st[:, 1].sum()), int(st[:, 11].sum()), int(st[:, 12].sum())

    for w in range(warmup):
        generation(1000 + w)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    produced = tests = accepted = nsteps = 0
    for k in range(steps):
        s_, p, t, a = generation(2000 + k)
        nsteps += s_
        produced += p
        tests += t
        accepted += a
        if early_exit_threshold is not None:
            exits += eng.exit_counts().sum(axis=0)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    seq0 = None
    if keep_seq0 > 0:
        seq0 = (eng.tokens()[0][:keep_seq0], eng.token_kinds()[0][:keep_seq0])
    out = {"value": round(produced / elapsed, 1), "unit": "tokens/s",
           "ms_per_generation": round(elapsed / steps * 1e3, 2),
           "pulse_steps_per_generation": round(nsteps / steps, 1),
           "acceptance_rate": round(accepted / tests, 4) if tests else None,
           "prefill_ms_first_call": round(prefill_s * 1e3, 1)}
    if early_exit_threshold is not None:
        out["exits_per_pulse"] = exits.tolist()
    if draft_len > 0 and produced > accepted:
        out["tokens_per_round"] = round(produced / (produced - accepted), 3)
    if seq0 is not None:
        out["seq0_tokens"], out["seq0_kinds"] = seq0
    log(f"{label}: {steps} timed generations, {produced} tokens in {elapsed:.3f}s, "
        f"acceptance {accepted}/{tests}")
    if profile:
        prof, bytes_by_class, psteps = profile_generation(eng, cfg, es, 3000)
        pair_ms, pair_n = prof.pop("event_pair")
        net = {k: v for k, v in prof.items() if v[1]}
        dom = max(net, key=lambda k: net[k][0])
        ms, n = net[dom]
        per_launch = bytes_by_class[dom] / max(n, 1)
        avg_s = ms / max(n, 1) / 1e3
        all_bytes = sum(bytes_by_class.values())
        out["hbm_roofline_frac_generation"] = round(all_bytes / (elapsed / steps) / HBM_PEAK, 4)
        out["algorithmic_bytes_per_generation"] = int(all_bytes)
        out["roofline"] = {"bound": "hbm", "kernel": dom,
                           "achieved": round(per_launch / avg_s / 1e9, 1), "peak": 8000.0,
                           "unit": "GB/s", "frac": round(per_launch / avg_s / HBM_PEAK, 4),
                           "bytes_per_launch": int(per_launch),
                           "avg_launch_us": round(avg_s * 1e6, 2),
                           "empty_event_pair_us": round(pair_ms / max(pair_n, 1) * 1e3, 2)}
        if trace_path:
            trace_fraction(out["roofline"], dom, trace_path)
        if traffic_path:
            tb = recorded_traffic(["class:" + dom], traffic_path)
            out["roofline"]["traffic"] = round(tb / 1e6, 3) if tb else None
            out["roofline"]["traffic_unit"] = ("MB per launch (rocprofv3 FETCH_SIZE + "
                                               "WRITE_SIZE, copy-calibrated, averaged over "
                                               "every launch of the class)")
        out["kernel_profile"] = {
            k: {"ms": round(v[0], 3), "launches": v[1], "us_per_launch": round(v[0] / v[1] * 1e3, 2),
                "GB_per_s": round(bytes_by_class[k] / max(v[0], 1e-9) / 1e6, 1)}
            for k, v in net.items()}
    eng.close()
    return out


def early_exit_run(model, cfg, prompts, args) -> dict:
    """The headline workload with the reference's adaptive early exit
    (set_early_exit_threshold, src/infer.py:536-547): plain decoding without and with the
    exit, and the self-speculative schedule with it (only accepted drafts can exit there,
    as in the reference), each one timed generation after a warm one."""
    kw = dict(steps=1, warmup=1, profile=False)
    thr = args.early_exit_threshold
    sampling = (args.temperature, args.top_p, args.repetition_penalty)
    plain = run_workload(model, cfg, prompts, args.new_tokens, *sampling, speculative=False,
                         label="plain", **kw)
    plain_ee = run_workload(model, cfg, prompts, args.new_tokens, *sampling, speculative=False,
                            early_exit_threshold=thr, label="plain early exit", **kw)
    spec_ee = run_workload(model, cfg, prompts, args.new_tokens, *sampling,
                           early_exit_threshold=thr, label="self-speculative early exit", **kw)
    return {"threshold": thr,
            "note": "random-init weights: the top-1 probability of every pulse-0 pass lies "
                    "between 0.99 and 0.999 (the tied-embedding self-logit dominates), so at "
                    "this threshold every eligible token leaves after pulse 0",
            "plain": {k: plain[k] for k in ("value", "unit", "pulse_steps_per_generation")},
            "plain_early_exit": {k: plain_ee[k] for k in ("value", "unit",
                                                          "pulse_steps_per_generation",
                                                          "exits_per_pulse")},
            "self_speculative_early_exit": {k: spec_ee[k] for k in (
                "value", "unit", "pulse_steps_per_generation", "acceptance_rate",
                "exits_per_pulse")}}


def _cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            return next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        return ""


def cpu_baseline(cfg, state, c2_prompts, c2_new, temperature, top_p, rp, c1_prompt, c1_new,
                 c2_seqs=(0, 15), c1_block=(), replays=()):
    """The oracle (PyTorch CPU restatement of src/infer.py, pinned to the reference by the
    golden vectors) on this host's cores: sequences c2_seqs of the headline workload in bf16
    one after another, as the batch-1 reference path runs them (sampled self-speculative,
    c2_new tokens after each prefill; the oracle's own acceptance rate beside the expected
    one), and c1 exactly (fp32, batch 1, greedy self-speculative, c1_new tokens), whose id
    stream the GPU run is checked against.

    As the checker of the GPU run it also computes: the draft-block restatement's greedy
    c1 streams (``block_speculative_ids``; c1_block: (name, draft length, repetition
    penalty, tokens) tuples), and for each entry of replays (name, prompt, emitted tokens,
    their kinds, draft length, temperature, tokens of the whole generation) the oracle's
    acceptance probabilities of the entry's draft tests replayed along its emitted stream
    (``replay_acceptance`` / ``replay_block_acceptance``), with the accepted count."""
    import torch

    from oracle import pulsar_ref as R

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    eng = R.load_ref(cfg, state, torch.bfloat16, stop_ids=set())
    torch.manual_seed(0)
    n = 0
    prefill_s = decode_s = 0.0
    acc = tests = 0
    p_acc = []
    for b in c2_seqs:
        stats = {}
        gen = eng.self_speculative_ids(c2_prompts[b], c2_new, temperature, top_p, rp,
                                       stats=stats)
        t0 = time.perf_counter()
        next(gen)  # the prefill and the first token
        t1 = time.perf_counter()
        n += len(list(gen))
        t2 = time.perf_counter()
        prefill_s += t1 - t0
        decode_s += t2 - t1
        acc += stats.get("accepted", 0)
        tests += stats.get("tests", 0)
        p_acc += stats.get("p_accept", [])
    ref1 = R.load_ref(cfg, state, torch.float32, stop_ids=set())
    g1 = ref1.self_speculative_ids(c1_prompt, c1_new, 0.0, 1.0, rp)
    u0 = time.perf_counter()
    c1_ids = [next(g1)]
    u1 = time.perf_counter()
    c1_ids += list(g1)
    u2 = time.perf_counter()
    seqs = " and ".join(str(b) for b in c2_seqs)
    blocks = {}
    for name, g_, rp_, n_ in c1_block:
        blocks[name] = list(ref1.block_speculative_ids(c1_prompt, n_, 0.0, 1.0, rp_, g_))
    rep_out = {}
    for name, prompt, toks, kinds, g_, temp_, total in replays:
        v0 = time.perf_counter()
        if g_ > 0:
            rep = R.replay_block_acceptance(eng, prompt, toks, kinds, temp_, top_p, rp, g_,
                                            max_new=total)
        else:
            rep = R.replay_acceptance(eng, prompt, toks, kinds, temp_, top_p, rp)
        ps = [p for p, _ in rep]
        rep_out[name] = {"tests": len(rep), "accepted": int(sum(a for _, a in rep)),
                         "expected_accepted": round(float(sum(ps)), 3),
                         "expected_acceptance": round(float(sum(ps) / len(ps)), 4) if ps else None,
                         "replayed_tokens": len(toks),
                         "s": round(time.perf_counter() - v0, 1)}
    return {
        "value": round(n / decode_s, 3) if n else None,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle in bf16 on sequences {seqs} of the headline workload, one after "
                   f"the other: {len(c2_prompts[0])}-token prompts prefilled in "
                   f"{prefill_s:.1f}s together (untimed), then {n} sampled self-speculative "
                   f"tokens after the first tokens in {decode_s:.1f}s; the reference path is "
                   f"batch 1, so the whole batch decodes at this rate; cpu "
                   f"'{_cpu_model_name()}', torch {torch.__version__}"),
        "acceptance_rate": round(acc / tests, 4) if tests else None,
        "acceptance_expected": round(sum(p_acc) / len(p_acc), 4) if p_acc else None,
        "tests": tests,
        "c1": {"workload": f"fp32, batch 1, {len(c1_prompt)}-token prompt, greedy "
                           f"self-speculative, {c1_new} new tokens",
               "value": round((len(c1_ids) - 1) / (u2 - u1), 3), "unit": "tokens/s",
               "prefill_and_first_token_s": round(u1 - u0, 2), "ids": c1_ids},
        "c1_block_ids": blocks,
        "acceptance_replay": rep_out,
    }


def op_surface_bench(cfg, reps: int = 20) -> dict:
    """Secondary figure for the pulsar_cuda op surface (the drop-in for src/model.py's fused
    functions): each forward op at a training micro-batch of 8 x 2048 tokens in bf16,
    HIP-event timed on the current stream over `reps` graph-replayed calls after 3 warm
    ones, with its algorithmic bytes (every input read once, every output written once)
    against the HBM peak."""
    import torch

    import pulsar_cuda as pc

    dev, bf = "cuda", torch.bfloat16
    B, T, D, H, Hkv = 8, 2048, cfg.d_model, cfg.n_heads, cfg.n_kv_heads
    E, K, ds = cfg.n_routed_experts, cfg.top_k, cfg.d_shared
    N = B * T
    g = torch.Generator(device=dev).manual_seed(0)

    def rnd(*shape, dtype=bf):
        return torch.randn(*shape, generator=g, device=dev).to(dtype)

    x = rnd(B, T, D)
    w = torch.rand(D, generator=g, device=dev) + 0.5
    qkv = rnd(B, T, (H + 2 * Hkv) * 64)
    q = qkv[..., : H * 64].view(B, T, H, 64).transpose(1, 2)
    wq = torch.rand(H, 64, generator=g, device=dev) + 0.5
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2, device=dev).float() / 64))
    f = torch.outer(torch.arange(T, device=dev).float(), inv)
    cos, sin = f.cos().contiguous(), f.sin().contiguous()
    attn = rnd(B, H, T, 64)
    gl = rnd(B, T, H, dtype=torch.float32)
    cw = rnd(D, 4, dtype=torch.float32) * 0.3
    gu = rnd(N, 2 * ds)
    logits = rnd(N, E) * 2
    bias = torch.zeros(E, device=dev)
    idx, tw, _, _ = pc.moe_router_topk_forward(logits, bias, K, 1e-3)
    flat = idx.reshape(-1).contiguous()
    C = int(-(-N * K * 1.25 // E))
    slots, counts = pc.moe_slots_from_order(flat, torch.argsort(flat, stable=True), E, C)
    slots = slots.view(N, K).contiguous()
    xr = x.view(N, D)
    kept = int((slots >= 0).sum())
    eo = rnd(E, C, D)
    sh = rnd(N, D)
    es = 2
    ops = {
        "rmsnorm": (lambda: pc.rmsnorm_forward(x, w, 1e-6), 2 * N * D * es + N * 4 + D * 4),
        "qk_rmsnorm_rope": (lambda: pc.qk_rmsnorm_rope_forward(q, wq, cos, sin, T, 1e-6),
                            2 * N * H * 64 * es + N * H * 4 + 2 * T * 32 * 4 + H * 64 * 4),
        "fused_attn_gate": (lambda: pc.fused_attn_gate_forward(attn, gl),
                            2 * N * H * 64 * es + N * H * 4),
        "causal_conv1d_k4": (lambda: pc.causal_depthwise_conv1d_k4_forward(x, cw),
                             2 * N * D * es + D * 16),
        "fused_swiglu": (lambda: pc.fused_swiglu_forward(gu, ds), 3 * N * ds * es),
        "moe_router_topk": (lambda: pc.moe_router_topk_forward(logits, bias, K, 1e-3),
                            N * E * es + N * K * (8 + 2)),
        "moe_dispatch": (lambda: pc.moe_dispatch_forward(xr, idx, slots, E, C, counts),
                         N * D * es + E * C * D * es + N * K * 12),
        "moe_combine": (lambda: pc.moe_combine_forward(eo, idx, tw, slots, sh),
                        kept * D * es + 2 * N * D * es + N * K * 14),
    }
    out = {}
    for name, (fn, nbytes) in ops.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        # device time: `reps` calls captured in one graph and replayed, so the host's
        # per-call cost (argument checks, output allocation) is not in the figure;
        # `us_eager` is the same calls launched one by one
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        graph.replay()
        t1.record()
        t1.synchronize()
        us = t0.elapsed_time(t1) / reps * 1e3
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        t1.synchronize()
        us_eager = t0.elapsed_time(t1) / reps * 1e3
        del graph
        out[name] = {"us": round(us, 2), "us_eager": round(us_eager, 2), "bytes": int(nbytes),
                     "GB_per_s": round(nbytes / us / 1e3, 1),
                     "hbm_frac": round(nbytes / (us * 1e-6) / HBM_PEAK, 4)}
    return {"workload": f"bf16, {B} x {T} tokens, d_model {D}, {H} heads of 64, {E} experts "
                        f"top-{K} (capacity {C}), shared d_ff {ds}", "ops": out}


def kv_footprint(cfg) -> dict:
    """KV-cache bytes at batch 1 in bf16 for 1k-32k contexts: the engine's allocation beside the
    reference's analytic unified-cache figure (src/infer.py:834-846)."""
    from pulsar_engine import traffic

    out = {}
    for ctx in (1024, 4096, 8192, 16384, 32768):
        e = traffic.kv_cache_bytes(cfg, 1, ctx)
        out[str(ctx)] = {"engine_MB": round(e["total"] / 1e6, 1),
                         "reference_MB": round(traffic.reference_unified_kv_bytes(ctx) / 1e6, 1),
                         "rewind_copy_MB": round(e["rewind_copy"] / 1e6, 1)}
    return out


def run_c4(model, cfg, args, profile: bool = True, draft_block: bool = True) -> dict:
    """4 sequences of 32768 uniform-random prompt tokens, 512 new tokens, greedy (the
    configuration names no temperature): reference schedule, and the draft-block mode at
    the configuration's draft length 4 beside it."""
    import numpy as np

    from pulsar_engine import weights as W
    p4 = np.stack([W.uniform_ids(90 + b, "c4_prompt", 32768, cfg.vocab_size) for b in range(4)])
    c4 = run_workload(model, cfg, p4, 512, 0.0, 1.0, args.repetition_penalty, steps=1,
                      warmup=1, label="c4", profile=profile)
    c4["workload"] = ("Pulsar-283M bf16, batch 4, 32768-token uniform prompts, greedy "
                      "self-speculative decode of 512 tokens (reference schedule)")
    if draft_block:
        c4["draft_block_4"] = run_workload(model, cfg, p4, 512, 0.0, 1.0,
                                           args.repetition_penalty, steps=1, warmup=1,
                                           profile=False, draft_len=4, label="c4 draft-block 4")
    log(f"c4: {json.dumps({k: v for k, v in c4.items() if k != 'kernel_profile'})}")
    return c4


def run_c5(cfg, state, args, profile: bool = True, draft_block: bool = True,
           exact: bool = True) -> dict:
    """256 sequences of 512 Zipf(1.1) prompt tokens, router weights x4, greedy, 512 new
    tokens; reference schedule, and the draft-block mode at draft length 6 beside it."""
    import numpy as np
    import torch

    from pulsar_engine import weights as W
    from pulsar_engine.model import DeviceModel
    # the skewed-routing weights: synthetic_state(router_scale=4) without regenerating
    st5 = {k: (v * np.float32(4.0)).astype(np.float32) if k.endswith("router_weight") else v
           for k, v in state.items()}
    m5 = DeviceModel(cfg, st5, torch.bfloat16)
    p5 = np.stack([W.zipf_ids(5, f"c5_prompt_{b}", 512, cfg.vocab_size) for b in range(256)])
    c5 = {}
    if exact:
        c5 = run_workload(m5, cfg, p5, 512, 0.0, 1.0, args.repetition_penalty, steps=1,
                          warmup=1, label="c5", profile=profile)
        c5["workload"] = ("Pulsar-283M bf16 with router weights x4, batch 256, 512-token "
                          "Zipf(1.1) prompts, greedy self-speculative decode of 512 tokens "
                          "(reference schedule)")
    if draft_block:
        c5["draft_block_6"] = run_workload(m5, cfg, p5, 512, 0.0, 1.0, args.repetition_penalty,
                                           steps=1, warmup=1, profile=False, draft_len=6,
                                           label="c5 draft-block 6")
    log(f"c5: {json.dumps({k: v for k, v in c5.items() if k != 'kernel_profile'})}")
    del m5, st5
    torch.cuda.empty_cache()
    return c5


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--prompt-len", type=int, default=2048)
    ap.add_argument("--new-tokens", type=int, default=256)
    ap.add_argument("--temperature", type=float, default=0.8)
    ap.add_argument("--top-p", type=float, default=0.95)
    ap.add_argument("--repetition-penalty", type=float, default=1.15)
    ap.add_argument("--plain", action="store_true", help="plain decode instead of self-speculative")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-new-tokens", type=int, default=48,
                    help="tokens per sequence of the CPU baseline (first and last sequence)")
    ap.add_argument("--no-c1", action="store_true", help="skip the c1 run (fp32, batch 1)")
    ap.add_argument("--no-c4", action="store_true", help="skip the long-context workload")
    ap.add_argument("--no-c5", action="store_true", help="skip the high-batch workload")
    ap.add_argument("--draft-len", type=int, default=4,
                    help="draft length of the draft-block run (0 skips it)")
    ap.add_argument("--no-verify", action="store_true", help="skip the verify microbenchmark")
    ap.add_argument("--no-ops", action="store_true", help="skip the op-surface figures")
    ap.add_argument("--no-early-exit", action="store_true", help="skip the early-exit runs")
    ap.add_argument("--no-t1", action="store_true",
                    help="skip the headline workload at temperature 1.0 (acceptance below 1)")
    ap.add_argument("--t1-temperature", type=float, default=1.0)
    ap.add_argument("--replay-tokens", type=int, default=48,
                    help="tokens of sequence 0 along which the oracle replays acceptance")
    ap.add_argument("--early-exit-threshold", type=float, default=0.99)
    ap.add_argument("--only", choices=("c4", "c5", "c5d6", "c2d4"),
                    help="run only that workload, unprofiled (kernel traces)")
    ap.add_argument("--verify-only", action="store_true",
                    help="run only the verify microbenchmark (profiling)")
    ap.add_argument("--verify-batch", type=int, default=64)
    ap.add_argument("--verify-ctx", type=int, default=8192)
    ap.add_argument("--verify-tokens", type=int, default=5)
    ap.add_argument("--verify-reps", type=int, default=20)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run device-to-device copies of MIB MiB (HBM counter calibration)")
    ap.add_argument("--phase", choices=("decode", "prefill"), default="decode",
                    help="phase of the trace --rocprof-summary tabulates")
    ap.add_argument("--rocprof-summary", metavar="DIR",
                    help="print the decode kernel table of a rocprofv3 csv kernel trace and exit")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH", "WRITE", "FETCH_COPY", "WRITE_COPY"),
                    help="print calibrated HBM bytes per decode dispatch from rocprofv3 --pmc "
                         "FETCH_SIZE / WRITE_SIZE csv directories (bench, then copy runs) and exit")
    args = ap.parse_args()
    if args.rocprof_summary:
        print(rocprof_summary(args.rocprof_summary, args.phase))
        return 0
    if args.pmc_summary:
        print(pmc_summary(*args.pmc_summary, copy_mib=256))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the decode path shards by sequence; see DESIGN.md)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from pulsar_engine import traffic
    from pulsar_engine import weights as W
    from pulsar_engine.config import PulsarConfig
    from pulsar_engine.engine import HipEngine
    from pulsar_engine.model import DeviceModel

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.calibrate_copy:
        # a plain copy of known size: reads and writes exactly n bytes per launch
        n = args.calibrate_copy << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {n} bytes 5 times")
        return 0
    cfg = PulsarConfig()
    B, T, N = args.batch, args.prompt_len, args.new_tokens
    t0 = time.perf_counter()
    state = W.synthetic_state(cfg, seed=0)
    log(f"weights generated in {time.perf_counter() - t0:.1f}s")
    model = DeviceModel(cfg, state, torch.bfloat16,
                        rope_len=max(cfg.max_seq_len, T + N + 16, args.verify_ctx + 32))
    es = 2
    if args.verify_only:
        vr = verify_microbench(model, cfg, es, args)
        print(json.dumps({"verify": vr}), flush=True)
        return 0
    if args.only == "c4":
        print(json.dumps({"c4": run_c4(model, cfg, args, profile=False, draft_block=False)}),
              flush=True)
        return 0
    if args.only == "c5":
        print(json.dumps({"c5": run_c5(cfg, state, args, profile=False, draft_block=False)}),
              flush=True)
        return 0
    if args.only == "c5d6":
        print(json.dumps({"c5": run_c5(cfg, state, args, profile=False, exact=False)}),
              flush=True)
        return 0
    prompts = np.stack([W.uniform_ids(0, f"bench_prompt_{b}", T, cfg.vocab_size) for b in range(B)])
    if args.only == "c2d4":
        print(json.dumps({"c2_draft_block": run_workload(
            model, cfg, prompts, N, args.temperature, args.top_p, args.repetition_penalty,
            args.steps, args.warmup, es, profile=False, draft_len=max(args.draft_len, 1),
            label="c2 draft-block")}), flush=True)
        return 0
    eng = HipEngine(model, batch=B, max_prompt=T, max_new=N, speculative=not args.plain,
                    temperature=args.temperature, top_p=args.top_p,
                    repetition_penalty=args.repetition_penalty, stop_ids=[], seed=1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.prefill(prompts)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"prefill {B}x{T} in {prefill_s:.3f}s (first call)")
    # a second prefill of the same prompts, warm: the wall time of the whole call
    # (host-to-device copy of the ids included), with the kernels it launches
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.prefill(prompts)
    torch.cuda.synchronize()
    prefill_warm_s = time.perf_counter() - t0
    pf = traffic.prefill_flops(cfg, B, T)
    prefill = {"ms": round(prefill_warm_s * 1e3, 2),
               "prompt_tokens_per_s": round(B * T / prefill_warm_s, 1),
               "bound": "mfma", "achieved": round(pf["total"] / prefill_warm_s / 1e12, 1),
               "peak": 2500.0, "unit": "TFLOP/s",
               "frac": round(pf["total"] / prefill_warm_s / MFMA_BF16_PEAK, 4),
               "flops": int(pf["total"]), "first_call_ms": round(prefill_s * 1e3, 1)}
    log(f"prefill {B}x{T} warm in {prefill_warm_s * 1e3:.1f} ms: {json.dumps(prefill)}")

    def generation(seed: int) -> tuple[int, int, int, int]:
        eng.rewind(seed)
        steps = eng.run(check_every=16)
        st = eng.state()
        return steps, int(st[:, 1].sum()), int(st[:, 11].sum()), int(st[:, 12].sum())

    for w in range(args.warmup):
        generation(1000 + w)
        log(f"warmup {w + 1}/{args.warmup} done")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    produced = tests = accepted = graph_steps = 0
    for k in range(args.steps):
        s, p, t, a = generation(2000 + k)
        produced += p
        tests += t
        accepted += a
        graph_steps += s
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    value = produced / elapsed
    log(f"timed {args.steps} generations: {produced} tokens in {elapsed:.3f}s, "
        f"{graph_steps} pulse steps, acceptance {accepted}/{tests}")

    roofline = None
    step_frac = None
    prof_detail = None
    if not args.no_profile:
        prof, bytes_by_class, psteps = profile_generation(eng, cfg, es, 3000)
        # Spans are kernel time plus what an event pair adds around a launch (under 1 us
        # with fence-free timing events, against the kernel trace). An empty pair, which
        # costs more than the overhead it adds around a kernel, is reported, not subtracted.
        pair_ms, pair_n = prof.pop("event_pair")
        pair = pair_ms / max(pair_n, 1)
        net = {k: v for k, v in prof.items() if v[1]}
        tot_ms = sum(v[0] for v in net.values())
        dom = max(net, key=lambda k: net[k][0])
        ms, n = net[dom]
        per_launch = bytes_by_class[dom] / max(n, 1)
        avg_s = ms / max(n, 1) / 1e3
        achieved = per_launch / avg_s
        traffic_b = recorded_traffic(["class:" + dom])
        roofline = {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": 8000.0,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                    "traffic": round(traffic_b / 1e6, 3) if traffic_b else None,
                    "traffic_unit": "MB per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                    "copy-calibrated, averaged over every launch of the "
                                    "class)",
                    "kernel": dom,
                    "bytes_per_launch": int(per_launch), "avg_launch_us": round(avg_s * 1e6, 2),
                    "empty_event_pair_us": round(pair * 1e3, 2)}
        trace_fraction(roofline, dom, DECODE_TRACE_PROFILE)
        all_bytes = sum(bytes_by_class.values())
        # whole-generation algorithmic bytes against the graph-replayed generation time
        step_frac = (all_bytes / (elapsed / args.steps)) / HBM_PEAK
        prof_detail = {k: {"ms": round(v[0], 3), "launches": v[1],
                           "us_per_launch": round(v[0] / v[1] * 1e3, 2),
                           "GB_per_s": round(bytes_by_class[k] / max(v[0], 1e-9) / 1e6, 1)}
                       for k, v in net.items()}
        log(f"profiled generation: {psteps} steps, {tot_ms:.1f} ms in timed spans (empty event "
            f"pair {pair * 1e3:.2f} us), dominant {dom} {ms:.1f} ms")
        log("per-class: " + json.dumps(prof_detail))

    exact = {"schedule": "exact self-speculative: the reference's draft length 1 (one pulse-0 "
                         "draft per token, tested against the token's pulse-2 draw), the "
                         "next token's pulse-0 draft pipelined with the verify pulse",
             "value": round(value, 1), "unit": "tokens/s",
             "ms_per_generation": round(elapsed / args.steps * 1e3, 2),
             "pulse_steps_per_generation": round(graph_steps / args.steps, 1),
             "acceptance_rate": round(accepted / tests, 4) if tests else None,
             "hbm_roofline_frac_generation": round(step_frac, 4) if step_frac is not None else None,
             "roofline": roofline, "kernel_profile": prof_detail}
    block = None
    if args.draft_len > 0 and not args.plain:
        block = run_workload(model, cfg, prompts, N, args.temperature, args.top_p,
                             args.repetition_penalty, args.steps, args.warmup, es,
                             profile=not args.no_profile, draft_len=args.draft_len,
                             label=f"c2 draft-block {args.draft_len}",
                             traffic_path=BLOCK_TRAFFIC_PROFILE,
                             trace_path=BLOCK_TRACE_PROFILE if args.draft_len == 4 else None)
        block["schedule"] = (f"draft-block, draft length {args.draft_len}: up to "
                             f"{args.draft_len} pulse-0 drafts per round, one all-pulse verify "
                             "of the block, drafts accepted down the block by the reference's "
                             "equal-draw rule; block rows after the first attend the block's "
                             "same-pulse keys (the prefill rule), so this schedule is not "
                             "reference-exact (exact_schedule is)")
        log(f"draft-block run: {json.dumps({k: v for k, v in block.items() if k != 'kernel_profile'})}")
    head = block if block is not None else exact
    # the headline workload at a temperature where drafts are rejected (the random-init
    # model accepts every draft at 0.8): both schedules, one timed generation each, with
    # sequence 0's stream kept for the oracle's acceptance replay in the CPU leg
    t1 = None
    if not args.no_t1 and not args.plain:
        t1 = {"workload": f"as the headline, temperature {args.t1_temperature}"}
        for name, g_ in (("exact_schedule", 0), (f"draft_block_{max(args.draft_len, 1)}",
                                                 max(args.draft_len, 1))):
            r = run_workload(model, cfg, prompts, N, args.t1_temperature, args.top_p,
                             args.repetition_penalty, 1, 1, es, profile=False, draft_len=g_,
                             label=f"t{args.t1_temperature} {name}",
                             keep_seq0=args.replay_tokens)
            t1[name] = {k: r.get(k) for k in ("value", "unit", "ms_per_generation",
                                              "pulse_steps_per_generation", "acceptance_rate",
                                              "tokens_per_round", "seq0_tokens", "seq0_kinds")}
            t1[name]["draft_len"] = g_
        log(f"temperature {args.t1_temperature}: " + json.dumps(
            {k: {x: y for x, y in v.items() if not x.startswith("seq0")}
             for k, v in t1.items() if isinstance(v, dict)}))
    early = None
    if not args.no_early_exit:
        early = early_exit_run(model, cfg, prompts, args)
        log(f"early exit: {json.dumps(early)}")
    verify = None
    if not args.no_verify:
        verify = verify_microbench(model, cfg, es, args)
        log(f"verify microbenchmark: {json.dumps(verify)}")
    # c1: fp32, batch 1, 128-token prompt, greedy self-speculative, 64 new tokens (the
    # reference's CPU-runnable case); its ids are checked against the oracle's below
    c1_prompt = W.uniform_ids(0, "prompt", 128, cfg.vocab_size)
    c1 = None
    if not args.no_c1:
        from pulsar_engine.engine import PulsarInferenceEngine

        m32 = DeviceModel(cfg, state, torch.float32)
        pe = PulsarInferenceEngine(m32)
        pe.generate_ids([c1_prompt.tolist()], max_new_tokens=64, temperature=0.0,
                        repetition_penalty=1.15, speculative=True, stop_ids=[])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        c1_ids = pe.generate_ids([c1_prompt.tolist()], max_new_tokens=64, temperature=0.0,
                                 repetition_penalty=1.15, speculative=True, stop_ids=[])[0]
        torch.cuda.synchronize()
        c1_s = time.perf_counter() - t0
        c1 = {"workload": "fp32, batch 1, 128-token uniform prompt, greedy self-speculative, "
                          "64 new tokens (prefill included)",
              "value": round(len(c1_ids) / c1_s, 1), "unit": "tokens/s",
              "ms_per_generation": round(c1_s * 1e3, 2), "ids": c1_ids}
        # the configuration's draft length 4 (draft-block schedule), at the headline penalty
        # and at penalty 10, where the greedy drafts are rejected now and then
        c1["draft_block_4"] = {}
        for name, rp_, n_ in (("rp1.15", 1.15, 64), ("rp10", 10.0, 32)):
            pe.generate_ids([c1_prompt.tolist()], max_new_tokens=n_, temperature=0.0,
                            repetition_penalty=rp_, speculative=True, stop_ids=[], draft_len=4)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ids_ = pe.generate_ids([c1_prompt.tolist()], max_new_tokens=n_, temperature=0.0,
                                   repetition_penalty=rp_, speculative=True, stop_ids=[],
                                   draft_len=4)[0]
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            tests_, acc_ = pe.last_engine.acceptance()
            c1["draft_block_4"][name] = {"repetition_penalty": rp_, "new_tokens": n_,
                                         "value": round(len(ids_) / dt, 1), "unit": "tokens/s",
                                         "acceptance_rate": round(acc_ / tests_, 4) if tests_ else None,
                                         "ids": ids_}
        # the reference's schedule at penalty 10 (stop ids 0 and 2) against the stream the
        # reference itself wrote for this prompt (tests/golden/full_fp32.npz)
        gold = np.load(os.path.join(ROOT, "tests", "golden", "full_fp32.npz"))
        assert np.array_equal(gold["prompt"], c1_prompt)
        rp10 = pe.generate_ids([c1_prompt.tolist()], max_new_tokens=32, temperature=0.0,
                               repetition_penalty=10.0, speculative=True, stop_ids=[0, 2])[0]
        c1["rp10_exact"] = {"repetition_penalty": 10.0, "new_tokens": 32, "stop_ids": [0, 2],
                            "ids": rp10, "identical_to_reference_golden":
                                rp10 == gold["greedy_rp10_spec_ids"].tolist()}
        for e_ in list(pe._engines.values()):
            e_.close()
        del pe, m32
        torch.cuda.empty_cache()
        log(f"c1: {c1['value']} tokens/s")
    c4 = None if args.no_c4 else run_c4(model, cfg, args)
    c5 = None if args.no_c5 else run_c5(cfg, state, args)
    ops = None
    if not args.no_ops:
        ops = op_surface_bench(cfg)
        log(f"op surface: {json.dumps(ops)}")
    cpu = None
    if not args.no_cpu_baseline:
        replays = []
        if t1 is not None:
            for name, v in t1.items():
                if isinstance(v, dict):
                    replays.append((name, prompts[0], v["seq0_tokens"], v["seq0_kinds"],
                                    v["draft_len"], args.t1_temperature, N))
        cpu = cpu_baseline(cfg, state, prompts, args.cpu_new_tokens, args.temperature,
                           args.top_p, args.repetition_penalty, c1_prompt, 64,
                           c2_seqs=sorted({0, len(prompts) - 1}),
                           c1_block=[] if c1 is None else [("rp1.15", 4, 1.15, 64),
                                                           ("rp10", 4, 10.0, 32)],
                           replays=replays)
        if c1 is not None:
            c1["token_identical_to_cpu_oracle"] = c1["ids"] == cpu["c1"]["ids"]
            for name, v in c1["draft_block_4"].items():
                v["token_identical_to_cpu_oracle_block"] = v["ids"] == cpu["c1_block_ids"][name]
        if t1 is not None:
            for name, rep in cpu["acceptance_replay"].items():
                t1[name]["oracle_replay_seq0"] = rep
        cpu.pop("c1_block_ids", None)
        log(f"cpu baseline: {json.dumps({k: v for k, v in cpu.items() if k != 'c1'})}")
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_generation"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights (N(0,0.02)), uniform random prompt ids",
        "config": {
            "workload": f"Pulsar-283M bf16, batch {B}, {T}-token prompts, sampled "
                        f"{'plain' if args.plain else 'self-speculative'} decode of {N} tokens",
            "batch": B, "prompt_len": T, "new_tokens": N, "temperature": args.temperature,
            "top_p": args.top_p, "repetition_penalty": args.repetition_penalty,
            "draft_len": args.draft_len if block is not None else (0 if args.plain else 1),
            "schedule": "plain" if args.plain else head["schedule"],
            "stop_ids": "disabled",
            "reference_exact": block is None,
        },
        "acceptance_rate": head["acceptance_rate"],
        "tokens_per_round": head.get("tokens_per_round"),
        "prefill": prefill,
        "hbm_roofline_frac_generation": head.get("hbm_roofline_frac_generation"),
        "roofline": head.get("roofline"),
        "cpu_baseline": cpu,
        "kernel_profile": head.get("kernel_profile"),
        "exact_schedule": exact if block is not None else None,
        "departure_from_reference_decode": None if block is None else {
            "what": "max|logits - reference decode_step logits| / max|reference| of the "
                    "verify's last-pulse rows 1..G against sequential decoding of the same "
                    "tokens (row 0 is identical); full-size model, 40-token prompt, "
                    "G = 4 and 6",
            "fp32": [1.6e-3, 6.3e-3], "bf16": [4.7e-3, 6.6e-3], "bound": 2e-2,
            "measured_by": "tests/test_oracle_block.py::"
                           "test_block_rows_depart_from_the_reference_decode_within_bound"},
        "temperature_1": t1,
        "verify": verify,
        "c1": c1,
        "c4": c4,
        "c5": c5,
        "kv_cache_batch1_bf16": kv_footprint(cfg),
        "early_exit": early,
        "op_surface": ops,
    }
    # id lists go to the log; the line keeps their checks. The objects a reader of the line's
    # end needs most (schedules, acceptance at temperature 1, c1 checks) come last.
    if c1 is not None:
        log("c1 ids: " + json.dumps({"exact": c1.pop("ids"), "rp10_exact": c1["rp10_exact"].pop("ids"),
                                     **{f"draft_block_4_{k}": v.pop("ids")
                                        for k, v in c1["draft_block_4"].items()}}))
    if t1 is not None:
        for name, v in t1.items():
            if isinstance(v, dict):
                log(f"temperature {args.t1_temperature} {name} sequence 0: "
                    f"{json.dumps({'tokens': v.pop('seq0_tokens'), 'kinds': v.pop('seq0_kinds')})}")
    if exact is not None and block is not None:
        line["exact_schedule_kernel_profile"] = exact.pop("kernel_profile", None)
    for k in ("verify", "c4", "c5", "c1", "exact_schedule", "departure_from_reference_decode",
              "temperature_1"):
        line[k] = line.pop(k)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
