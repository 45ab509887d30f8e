"""Benchmark of the decision-path pass on one MI355X.

Workload (the metric's configuration): a
Gemma-3-270M-shaped decoder with seeded Q4_0 weights and a 25,000-row
vocabulary, one 2,000-token state plus 12 question branches of 32 tokens
in one block-causal pass, label readout at each branch's last position:
the 26 label logits and the log-sum-exp of the full 25,000-wide row, what
the reference's Readout::distribution takes from the row
(crates/omg-core/src/readout.rs:124-146).  Each timed step launches the
whole pass: eagerly (one launch per kernel) and as a replay of the pass
captured once into a HIP graph; `value` takes the faster, both are
reported under `launch`.  A step is one cold pass (state + branches, T = 2,384) with
the token ids and metadata already in HBM; the warm pass (branches only on
the resident state, T = 384) and the API wall times (host upload and
readback included: `api_ms` cold / warm are medians of the C ABI call on
arguments marshalled once, `python_*` one call through the Python
wrapper) are reported beside it.

`--config c4` measures BASELINE.json configs[3] instead: the Laya encoder
path over 192 sequences of 256 tokens (see bench_encoder).  `--config e2b`
measures the reference's published Gemma 4 workload (E2B-shaped Q4_0, 12
questions over a 2,000-token state; see bench_gemma4) as cold and warm
latency against the published figures.

Prints one JSON line (see the repository's driver contract).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "questions/sec + state prefill tok/s (Gemma-3-270M Q4_0, 2k state, 12 Qs), 1 GPU"
PEAK_F16_TFLOPS = 2500.0   # MI355X dense FP16/BF16 MFMA
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
SEED = 0x5EED


def linear_macs_per_token(cfg) -> dict:
    d, ff, H, KV, hd = cfg["d"], cfg["ff"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    return {"mm_qkv": (H + 2 * KV) * hd * d, "mm_o": d * H * hd, "mm_gate_up": 2 * ff * d, "mm_down": d * ff}


def visible_pairs(prefix: int, nb: int, bt: int, window: int, layers: int, pattern: int = 6,
                  skip_last: bool = False) -> int:
    """Query-key pairs the block-causal mask admits over all layers (the
    attention FLOP count is 4 * heads * head_dim per pair); skip_last
    leaves the last layer out."""
    total = 0
    for layer in range(layers - 1 if skip_last else layers):
        w = window if (layer + 1) % pattern != 0 else 0
        for q in range(prefix):
            total += min(q + 1, w) if w else q + 1
        for j in range(bt):
            qp = prefix + j
            vis_prefix = prefix if not w else max(0, min(prefix, prefix - (qp - w + 1)))
            vis_own = j + 1 if not w else min(j + 1, w)
            total += nb * (vis_prefix + vis_own)
    return total


def storage_bytes_per_elem(dtype) -> float:
    """Q4_0 / Q8_0 / F16 bytes per weight (codes + block scales)."""
    import grande_amd as g

    return {g.Q4: 18 / 32, g.Q8: 34 / 32, g.F16: 2.0}[dtype]


def pass_bytes(cfg, dtype, prefix: int, nb: int, bt: int, pattern: int = 6) -> dict:
    """Algorithmic HBM bytes of one pass over a resident prefix: every
    linear weight once, the token embedding once (the full-row log-sum-exp
    reads every logit), and each layer's K and V rows that some query of
    the pass can see (global layers: the whole prefix and the branches;
    sliding layers: the last `window` prefix keys and the branches),
    f16 K / V of kv_heads x head_dim per key."""
    d, ff, H, KV, hd, L = cfg["d"], cfg["ff"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["layers"]
    per_tok = sum(linear_macs_per_token(cfg).values())
    w = per_tok * L * storage_bytes_per_elem(dtype)
    emb = cfg["vocab"] * d * storage_bytes_per_elem(dtype)
    kv = 0
    for layer in range(L):
        win = cfg["window"] if (layer + 1) % pattern != 0 else 0
        keys = (min(prefix, win) if win else prefix) + nb * bt
        kv += keys * KV * hd * 2 * 2
    return {"weights": w, "embedding": emb, "kv": kv, "total": w + emb + kv}


def kernel_bytes(cfg, dtype, m: int) -> dict:
    """Algorithmic HBM bytes of one launch of each linear product and of the
    residual norm over m rows: the weight once, the f16 activations in, the
    outputs (f32 split-K partials of the o / down products, two at these
    shapes; f16 q rows and K / V cache rows; f16 gated activations; the
    norm's stream read and written with its f16 output)."""
    d, ff, H, KV, hd = cfg["d"], cfg["ff"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    s = storage_bytes_per_elem(dtype)

    def splits(k, n):  # the engine's K split of the o / down products at these shapes
        return 2 if n <= 1280 and k >= 1024 else 1

    return {
        "mm_qkv": (H + 2 * KV) * hd * d * s + m * d * 2 + m * (H + 2 * KV) * hd * 2,
        "mm_o": d * H * hd * s + m * H * hd * 2 + m * d * 4 * splits(H * hd, d),
        "mm_gate_up": 2 * ff * d * s + m * d * 2 + m * ff * 2,
        "mm_down": d * ff * s + m * ff * 2 + m * d * 4 * splits(ff, d),
        "norm": m * d * (4 * 2 + 4 * 2 + 2),
    }


class MallFlush:
    """Evicts the MALL between timed reps: one device-to-device copy of
    `nbytes` (reads nbytes, writes nbytes), through the HIP runtime the
    engine's library is linked against (a second runtime in the process,
    such as torch's, would not see the GPU)."""

    def __init__(self, nbytes: int):
        import ctypes

        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.nbytes = nbytes
        self.src, self.dst = ctypes.c_void_p(), ctypes.c_void_p()
        for ptr in (self.src, self.dst):
            if self.hip.hipMalloc(ctypes.byref(ptr), ctypes.c_size_t(nbytes)) != 0:
                raise RuntimeError("hipMalloc failed")
        self.hip.hipMemset(self.src, 1, ctypes.c_size_t(nbytes))
        self.hip.hipDeviceSynchronize()

    def __call__(self):
        import ctypes

        if self.hip.hipMemcpy(self.dst, self.src, ctypes.c_size_t(self.nbytes), 3) != 0:  # device to device
            raise RuntimeError("hipMemcpy failed")
        self.hip.hipDeviceSynchronize()

    def close(self):
        self.hip.hipFree(self.src)
        self.hip.hipFree(self.dst)


def profiled_traffic(config: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (profiles/<config>_<kernel>_traffic.md, a line "traffic_bytes_per_launch:
    N"), or None where there is none."""
    path = ROOT / "profiles" / f"{config}_{kernel}_traffic.md"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo, as lscpu reports it) and
    the logical CPUs this process may run on."""
    name = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return f"{name}; {len(os.sched_getaffinity(0))} logical CPUs available"


def c_api_ms(eng, groups, labels, reps: int = 15) -> dict:
    """Medians of the C ABI's omg_evaluate_groups on arguments marshalled
    once (what a compiled caller pays: host ids in, label logits and the
    log-sum-exp out, synchronised): cold with the resident prefix evicted
    first, warm on the resident state."""
    import ctypes as C
    from grande_amd import Want, _lib as L
    from grande_amd.engine import _CGroups, _u32
    cg, lab = _CGroups(groups), _u32(labels)
    rows = sum(len(b.want) for gr in groups for b in gr.branches)
    out = np.zeros((rows, lab.size + 1), np.float32)
    src = (C.c_int * len(groups))()
    lib = L.lib()

    def call() -> float:
        t = time.perf_counter()
        L.check(lib.omg_evaluate_groups(eng._h, cg.arr, cg.n, int(Want.LABELS_LSE),
                                        lab.ctypes.data_as(C.POINTER(C.c_uint32)), lab.size,
                                        out.ctypes.data_as(C.POINTER(C.c_float)), out.size, src))
        return time.perf_counter() - t

    cold, warm = [], []
    for _ in range(reps):
        eng.evict_resident()
        cold.append(call())
        warm.append(call())
    return {"cold": round(float(np.median(cold)) * 1e3, 3), "warm": round(float(np.median(warm)) * 1e3, 3),
            "reps": reps, "calls": "C ABI, arguments marshalled once"}


def small_batch_leg(eng, prefix, branch, labels, mc, dtype, P: int, BT: int, reps: int, no_graph: bool) -> dict:
    """One branch of BT tokens on the resident P-token state, every rep
    preceded by a device-to-device copy of 512 MiB (1 GiB of traffic, twice
    the 256 MB MALL) so weights, embedding and K/V come from HBM; one graph
    replay per rep, timed to its end.  Per-kernel HIP-event times of three
    more flushed reps (eager launches), and each product's algorithmic bytes
    and the rate its interval implies."""
    from grande_amd import Group, Want

    one = [branch]
    eng.evaluate(prefix, one, Want.LABELS_LSE, labels)  # the state becomes resident
    eng.prepare([Group(prefix, one)], Want.LABELS_LSE, labels, first_resident=True)
    if not no_graph:
        eng.graph(True)
    eng.launch()
    eng.sync()
    flush = MallFlush(512 << 20)
    times = []
    for _ in range(reps):
        flush()
        t = time.perf_counter()
        eng.launch()
        eng.sync()
        times.append(time.perf_counter() - t)
    eng.graph(False)
    eng.profile(True)
    for _ in range(3):
        flush()
        eng.launch()
        eng.sync()
    sprof = eng.profile_report()
    eng.profile(False)
    flush.close()
    sb = pass_bytes(mc, dtype, P, 1, BT)
    s_ms = float(np.median(times)) * 1e3
    gbs = sb["total"] / (s_ms * 1e-3) / 1e9
    small = {"branches": 1, "branch_tokens": BT, "reps": reps, "ms_median": round(s_ms, 4),
             "ms_min": round(min(times) * 1e3, 4), "mall_flush_bytes": 2 * flush.nbytes,
             "algorithmic_bytes": {k: int(v) for k, v in sb.items()}, "gb_per_s": round(gbs, 1),
             "hbm_peak_gb_per_s": HBM_PEAK_GBS, "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
             "kernels": {name: {"launches_per_step": n // 3, "avg_us": round(ms / n * 1e3, 2)}
                         for name, (n, ms) in sprof.items()}}
    # per-launch algorithmic bytes and rate of the products and the norm
    # (HIP-event intervals: each includes the dispatch gap before it)
    for name, nbytes in kernel_bytes(mc, dtype, BT).items():
        k = small["kernels"].get(name)
        if k and k["avg_us"] > 0:
            k["bytes"] = int(nbytes)
            k["gb_per_s"] = round(nbytes / (k["avg_us"] * 1e-6) / 1e9, 1)
            k["hbm_frac"] = round(k["gb_per_s"] / HBM_PEAK_GBS, 4)
    return small


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--small-reps", type=int, default=10,
                    help="reps of the small-batch leg (one branch on the resident state, MALL flushed)")
    ap.add_argument("--no-4b", action="store_true", help="skip the small-batch leg at the 4B shape (C5)")
    ap.add_argument("--no-graph", action="store_true",
                    help="eager launches only (no HIP graph capture or replay): for runs under rocprofv3, whose "
                         "kernel tracing faulted inside hipGraphLaunch")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 256 MiB device to device three times (calibrates the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this engine runs on one GPU (--gpus {args.gpus} requested); a state's branches would "
              "shard across GPUs by broadcasting the prefix K/V, which is not built.", file=sys.stderr)
        return 2

    if args.copy_probe:
        import torch

        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4, "copies": 3}))
        return 0

    if args.config == "c4":
        return bench_encoder(args)
    if args.config == "e2b":
        return bench_gemma4(args)

    import grande_amd as g
    from grande_amd import BranchTokens, Group, Want

    spec = g.BASELINE_CONFIGS[args.config]
    mc = spec["model"]
    wname = {g.Q4: "q4_0", g.Q8: "q8_0", g.F16: "f16"}[spec["dtype"]]
    size = {640: "270M", 1152: "1B", 2560: "4B"}.get(mc["d"], f"d{mc['d']}")
    shape = f"Gemma-3-{size}-shaped {wname.upper()}"
    cfg = g.config_json(**mc)
    P, NB, BT = spec["state"], spec["branches"], spec["branch_tokens"]
    T = P + NB * BT
    rng = np.random.default_rng(SEED)
    prefix = rng.integers(0, mc["vocab"], P).tolist()
    branches = [BranchTokens(rng.integers(0, mc["vocab"], BT).tolist(), [BT - 1]) for _ in range(NB)]
    labels = g.LABEL_IDS

    t0 = time.perf_counter()
    weights = g.Weights.synth(cfg, SEED, spec["dtype"], spec["dtype"])
    eng = g.Engine.new(weights, T + 64, max(64, NB))
    load_s = time.perf_counter() - t0

    # API passes (host ids in, label logits out): cold, then warm on the
    # resident state, then a state save / evict / restore round trip.  One
    # untimed cold and warm pair first: the first launch of each kernel
    # loads its code object.
    eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    eng.evict_resident()
    t = time.perf_counter()
    cold_rows = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    api_cold_ms = (time.perf_counter() - t) * 1e3
    t = time.perf_counter()
    warm_rows = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    api_warm_ms = (time.perf_counter() - t) * 1e3
    assert eng.prefix_source() == g.PrefixSource.RESIDENT
    c_api = c_api_ms(eng, [Group(prefix, branches)], labels)
    # (one untimed save and restore first: their first calls load the
    # gather / scatter kernels and touch the pinned staging pages)
    eng.restore_state(eng.save_state(prefix, "bench"), "bench")
    saves, restores = [], []
    for _ in range(5):  # medians of five round trips
        t = time.perf_counter()
        state = eng.save_state(prefix, "bench")
        saves.append(time.perf_counter() - t)
        eng.evict_resident()
        t = time.perf_counter()
        eng.restore_state(state, "bench")
        restores.append(time.perf_counter() - t)
    save_ms, restore_ms = float(np.median(saves)) * 1e3, float(np.median(restores)) * 1e3
    restored_rows = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    restored_equal = all(np.array_equal(a.rows[0], b.rows[0]) for a, b in zip(warm_rows, restored_rows))
    warm_equal_cold = max(float(np.max(np.abs(a.rows[0] - b.rows[0]))) for a, b in zip(cold_rows, warm_rows))

    def timed(first_resident: bool, steps: int, warmup: int, graph: bool = False) -> float:
        eng.prepare([Group(prefix, branches)], Want.LABELS_LSE, labels, first_resident=first_resident)
        for _ in range(warmup):
            eng.launch()
        if graph:
            eng.graph(True)  # the pass's launches captured once, replayed per step
            eng.launch()
        eng.sync()
        t = time.perf_counter()
        for _ in range(steps):
            eng.launch()
        eng.sync()
        return (time.perf_counter() - t) / steps

    eng.evict_resident()
    cold_eager_s = timed(False, args.steps, args.warmup)
    cold_graph_s = cold_eager_s if args.no_graph else timed(False, args.steps, args.warmup, graph=True)
    eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)  # leaves the state resident
    warm_eager_s = timed(True, args.steps, args.warmup)
    warm_graph_s = warm_eager_s if args.no_graph else timed(True, args.steps, args.warmup, graph=True)
    cold_s, warm_s = min(cold_eager_s, cold_graph_s), min(warm_eager_s, warm_graph_s)

    # Per-kernel HIP-event times over a second timed region of cold steps,
    # then of warm steps (the branches on the resident state).
    eng.profile(True)
    timed(False, args.steps, 0)
    prof = eng.profile_report()
    eng.profile(False)
    eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    eng.profile(True)
    timed(True, args.steps, 0)
    wprof = eng.profile_report()
    eng.profile(False)

    macs = linear_macs_per_token(mc)
    pairs = visible_pairs(P, NB, BT, mc["window"], mc["layers"])
    flops = {k: 2.0 * T * v for k, v in macs.items()}
    flops["attention"] = 4.0 * mc["heads"] * mc["head_dim"] * pairs / mc["layers"]
    if "attention_out" in prof:
        # The last layer past its q/k/v product ran for the answer rows only
        # (its launches are the *_out steps): the full-row launches are the
        # other layers', so the attention launch's average work is theirs.
        flops["attention"] = 4.0 * mc["heads"] * mc["head_dim"] * visible_pairs(
            P, NB, BT, mc["window"], mc["layers"], skip_last=True) / (mc["layers"] - 1)
    # Small-batch leg: one branch of BT tokens on the resident state, the
    # serving loop's common case.  Before every rep 1 GiB is read and
    # written, which evicts the 256 MB MALL, so the pass's weights, embedding
    # and K/V come from HBM; each rep is one graph launch, timed to its end.
    small = None
    if args.small_reps > 0:
        small = small_batch_leg(eng, prefix, branches[0], labels, mc, spec["dtype"], P, BT, args.small_reps,
                                args.no_graph)
    # The same leg at the 4B shape (C5: one 40-token branch over its
    # 8,000-token state), where the products are large enough to show an
    # HBM rate: 30 MB gate/up, 16 MB down per launch.
    small_4b = None
    if args.small_reps > 0 and args.config == "c2" and not args.no_4b:
        s5 = g.BASELINE_CONFIGS["c5"]
        m5 = s5["model"]
        cfg5 = g.config_json(**m5)
        P5, BT5 = s5["state"], s5["branch_tokens"]
        rng5 = np.random.default_rng(SEED + 5)
        prefix5 = rng5.integers(0, m5["vocab"], P5).tolist()
        branch5 = BranchTokens(rng5.integers(0, m5["vocab"], BT5).tolist(), [BT5 - 1])
        w5 = g.Weights.synth(cfg5, SEED + 5, s5["dtype"], s5["dtype"])
        eng5 = g.Engine.new(w5, P5 + BT5 + 64, 64)
        del w5
        small_4b = small_batch_leg(eng5, prefix5, branch5, labels, m5, s5["dtype"], P5, BT5, args.small_reps,
                                   args.no_graph)
        w5name = {g.Q4: "Q4_0", g.Q8: "Q8_0", g.F16: "F16"}[s5["dtype"]]
        small_4b["workload"] = f"c5: Gemma-3-4B-shaped {w5name}, one {BT5}-token branch on the resident " \
                               f"{P5}-token state"
        eng5.close()

    kernels = {}
    for name, (n, ms) in prof.items():
        avg_us = ms / n * 1e3
        entry = {"launches_per_step": n // args.steps, "avg_us": round(avg_us, 2),
                 "share": round(ms / sum(v[1] for v in prof.values()), 4)}
        if name in flops:
            tf = flops[name] / (avg_us * 1e-6) / 1e12
            entry.update(tflops=round(tf, 1), mfma_frac=round(tf / PEAK_F16_TFLOPS, 4))
        kernels[name] = entry
    dom = max((k for k in kernels if k in flops), key=lambda k: prof[k][1])
    dom_tf = kernels[dom]["tflops"]
    # the pass's algorithmic work (every layer, every row: the reference's
    # pass), and that of the full-row launches that ran (with the answer-row
    # last layer: its o, gate/up, down and attention on the 12 answer rows,
    # under 0.1% of the pass, are left out)
    total_flop = sum(2.0 * T * v for v in macs.values()) * mc["layers"] + 4.0 * mc["heads"] * mc["head_dim"] * pairs
    ran_flop = total_flop
    if "attention_out" in prof:
        ran_flop = (sum(2.0 * T * v for v in macs.values()) * (mc["layers"] - 1) + 2.0 * T * macs["mm_qkv"]
                    + 4.0 * mc["heads"] * mc["head_dim"] * visible_pairs(P, NB, BT, mc["window"], mc["layers"],
                                                                        skip_last=True))
    warm_flops = {k: 2.0 * NB * BT * v for k, v in macs.items()}
    wb = pass_bytes(mc, spec["dtype"], P, NB, BT)
    warm_pairs = visible_pairs(P, NB, BT, mc["window"], mc["layers"]) - visible_pairs(P, 0, BT, mc["window"], mc["layers"])
    warm_flop = sum(warm_flops.values()) * mc["layers"] + 4.0 * mc["heads"] * mc["head_dim"] * warm_pairs
    warm_kernels = {}
    for name, (n, ms) in wprof.items():
        avg_us = ms / n * 1e3
        entry = {"launches_per_step": n // args.steps, "avg_us": round(avg_us, 2),
                 "share": round(ms / sum(v[1] for v in wprof.values()), 4)}
        if name in warm_flops:
            entry["tflops"] = round(warm_flops[name] / (avg_us * 1e-6) / 1e12, 1)
        warm_kernels[name] = entry

    out = {
        "metric": METRIC if args.config == "c2" else f"questions/sec ({args.config}: {shape}), 1 GPU",
        "value": round(NB / cold_s, 2),
        "unit": "questions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(cold_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{wname} weights, f16 MFMA, f32 accumulate",
        "data": "synthetic (seeded random-init weights and token ids)",
        "config": {"workload": f"{args.config}: {shape}, vocab 25k, state {P} + {NB}x{BT} branches, "
                               "26 label logits + full-row log-sum-exp readout", "tokens": T, "state_tokens": P, "branches": NB,
                   "branch_tokens": BT},
        "launch": {"cold_eager_ms": round(cold_eager_s * 1e3, 4), "cold_graph_ms": round(cold_graph_s * 1e3, 4),
                   "warm_eager_ms": round(warm_eager_s * 1e3, 4), "warm_graph_ms": round(warm_graph_s * 1e3, 4),
                   "graphs": not args.no_graph},
        "cold_tok_per_s": round(T / cold_s, 1),
        "warm_ms": round(warm_s * 1e3, 4),
        "warm_questions_per_s": round(NB / warm_s, 2),
        "warm_tok_per_s": round(NB * BT / warm_s, 1),
        "api_ms": {**c_api, "python_cold": round(api_cold_ms, 3), "python_warm": round(api_warm_ms, 3),
                   "state_save": round(save_ms, 3),
                   "state_restore": round(restore_ms, 3), "state_bytes": len(state)},
        "restored_bit_equal": bool(restored_equal),
        "warm_vs_cold_max_abs_logit": warm_equal_cold,
        "pass_tflops": round(ran_flop / cold_s / 1e12, 2),
        "pass_tflops_algorithmic": round(total_flop / cold_s / 1e12, 2),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": dom_tf, "peak": PEAK_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(dom_tf / PEAK_F16_TFLOPS, 4),
                     "traffic": profiled_traffic(args.config, dom)},
        "kernels": kernels,
        "warm_kernels": warm_kernels,
        "warm_roofline": {"flop": warm_flop, "tflops": round(warm_flop / warm_s / 1e12, 2),
                          "mfma_frac": round(warm_flop / warm_s / 1e12 / PEAK_F16_TFLOPS, 4),
                          "algorithmic_bytes": int(wb["total"]), "gb_per_s": round(wb["total"] / warm_s / 1e9, 1),
                          "hbm_frac": round(wb["total"] / warm_s / 1e9 / HBM_PEAK_GBS, 4)},
        "small_batch": small,
        "small_batch_4b": small_4b,
        "load_s": round(load_s, 2),
    }

    if not args.no_cpu:
        import oracle

        model = oracle.Model(cfg, list(weights.tensors()))
        ids, pos, seq = oracle.pack_single(prefix, branches)
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        # Whole cold passes, repeated until about 10 s of CPU work (at most 30 passes).
        t = time.perf_counter()
        passes = 0
        while True:
            hidden = model.forward(ids, pos, seq)
            rows = np.stack([hidden[P + i * BT + BT - 1] for i in range(NB)])
            cpu_logits = model.logits(rows)
            lse = np.log(np.exp(cpu_logits - cpu_logits.max(1, keepdims=True)).sum(1)) + cpu_logits.max(1)
            cpu_logits = np.concatenate([cpu_logits[:, labels], lse[:, None]], 1)
            passes += 1
            if time.perf_counter() - t >= 10.0 or passes >= 30:
                break
        cpu_s = (time.perf_counter() - t) / passes
        dp, dmass, argmax_same = 0.0, 0.0, True
        cpu_full = model.logits(rows)
        for i in range(NB):
            got = cold_rows[i].rows[0]
            pg = oracle.softmax(got[:-1])
            _, pc, mass_c = oracle.label_readout(cpu_full[i], labels)
            mass_g = float(np.exp(oracle.log_sum_exp(got[:-1]) - float(got[-1])))
            dp = max(dp, float(np.max(np.abs(pg - pc))))
            dmass = max(dmass, abs(mass_g - mass_c))
            argmax_same &= int(np.argmax(pg)) == int(np.argmax(pc))
        out["cpu_baseline"] = {"value": round(NB / cpu_s, 4), "unit": "questions/s", "cores": threads,
                               "cpu_model": cpu_model(),
                               "kind": "port", "sample": f"{passes} full cold passes of the same workload ({T} tokens, "
                               f"{mc['layers']} layers) + label readout, f32 C restatement of the reference CPU "
                               f"forward, OpenMP; value from the mean pass", "seconds": round(cpu_s * passes, 3),
                               "gpu_speedup": round(cpu_s / cold_s, 1)}
        out["parity"] = {"max_abs_dprob_after_softmax": dp, "max_abs_dcandidate_mass": dmass,
                         "argmax_identical": bool(argmax_same), "tol": 2e-2}
    print(json.dumps(out))
    return 0


def encoder_seqs(spec, rng):
    """configs[3]'s requests: per question a 256-token sequence ([CLS] ...
    [SEP]) with one [MASK]; question types cycle choice / score / noul."""
    from grande_amd import laya as ly

    seqs = []
    for r in range(spec["requests"] * spec["questions"]):
        ids = rng.integers(5, spec["model"]["vocab"], spec["seq_len"]).tolist()
        ids[0], ids[-1] = 1, 2
        m = int(rng.integers(8, spec["seq_len"] - 8))
        ids[m] = 4
        seqs.append(ly.Sequence(ids, [m], r % 3))
    return seqs


def encoder_pairs(n: int, window: int) -> int:
    """Query-key pairs of one n-token sequence: all, or |i - j| <= window."""
    if not window:
        return n * n
    return sum(min(n, i + window + 1) - max(0, i - window) for i in range(n))


def gemma4_layer_shapes(mc) -> list[dict]:
    """Per layer: sliding, head_dim, own K/V, ff (model.rs:95-210)."""
    L, shared = mc["layers"], mc["shared_kv_layers"]
    out = []
    for i in range(L):
        s = mc["sliding"][i]
        out.append(dict(sliding=s, hd=mc["head_dim"] if s else mc["global_head_dim"], own_kv=i < L - shared,
                        ff=mc["ff"] * (2 if mc["double_wide_mlp"] and i >= L - shared else 1)))
    return out


def pairs_one_layer(prefix: int, bts: list, window: int) -> int:
    """Query-key pairs the block-causal mask admits on one layer (window 0
    = global) for one state and branches of lengths `bts`."""
    total = 0
    for q in range(prefix):
        total += min(q + 1, window) if window else q + 1
    for bt in bts:
        for j in range(bt):
            qp = prefix + j
            vis_prefix = prefix if not window else max(0, min(prefix, prefix - (qp - window + 1)))
            total += vis_prefix + (j + 1 if not window else min(j + 1, window))
    return total


def bench_gemma4(args) -> int:
    """The reference's published Gemma 4 workload (docs/comparison.md:92,
    116): E2B-shaped Q4_0, one 2,000-token state and 12 question branches
    (663 tokens), label readout at each branch's last position.  A step is
    one cold pass (T = 2,663) with the inputs in HBM; the warm pass
    (branches only on the resident state) beside it.  The published
    figures are wall-clock on an Apple M4 GPU; `vs_baseline` divides this
    latency by the cold one (lower is better)."""
    import grande_amd as g
    from grande_amd import BranchTokens, Group, Want

    spec = g.GEMMA4_CONFIGS[args.config]
    mc = spec["model"]
    cfg = g.gemma4_config_json(**mc)
    P, bts = spec["state"], spec["branch_tokens"]
    T = P + sum(bts)
    rng = np.random.default_rng(SEED)
    prefix = rng.integers(0, mc["vocab"], P).tolist()
    branches = [BranchTokens(rng.integers(0, mc["vocab"], bt).tolist(), [bt - 1]) for bt in bts]
    labels = g.LABEL_IDS
    t0 = time.perf_counter()
    eng = g.Engine.new(g.Weights.synth(cfg, SEED, spec["dtype"], spec["dtype"]), T + 64, 64)
    load_s = time.perf_counter() - t0
    eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)  # untimed: first launches load code objects
    eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    eng.evict_resident()
    t = time.perf_counter()
    cold_rows = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    api_cold_ms = (time.perf_counter() - t) * 1e3
    t = time.perf_counter()
    warm_rows = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    api_warm_ms = (time.perf_counter() - t) * 1e3
    warm_equal_cold = max(float(np.max(np.abs(a.rows[0] - b.rows[0]))) for a, b in zip(cold_rows, warm_rows))

    def timed(first_resident: bool, steps: int, warmup: int) -> float:
        eng.prepare([Group(prefix, branches)], Want.LABELS_LSE, labels, first_resident=first_resident)
        for _ in range(warmup):
            eng.launch()
        eng.sync()
        t = time.perf_counter()
        for _ in range(steps):
            eng.launch()
        eng.sync()
        return (time.perf_counter() - t) / steps

    eng.evict_resident()
    cold_s = timed(False, args.steps, args.warmup)
    eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    warm_s = timed(True, args.steps, args.warmup)
    eng.profile(True)
    timed(False, args.steps, 0)
    prof = eng.profile_report()
    eng.profile(False)

    shapes = gemma4_layer_shapes(mc)
    d, H, KV, Pl = mc["d"], mc["heads"], mc["kv_heads"], mc["per_layer_dim"]

    def layer_flop(s):
        return {"mm_qkv": 2.0 * T * d * (H + (2 * KV if s["own_kv"] else 0)) * s["hd"],
                "mm_o": 2.0 * T * d * H * s["hd"], "mm_gate_up": 4.0 * T * d * s["ff"],
                "mm_down": 2.0 * T * d * s["ff"],
                "attention": 4.0 * H * s["hd"] * pairs_one_layer(P, bts, mc["window"] if s["sliding"] else 0)}

    # The algorithmic work of the pass (every layer, every row: the
    # reference's), and that of the full-row launches that ran: with the
    # answer-row path (`*_out` steps) the layers after the last one that
    # writes K/V, and that layer past its q/k/v product, run on the 12
    # answer rows only (their work, under 0.1% of the pass, is left out).
    algo = {k: 0.0 for k in ("mm_qkv", "mm_o", "mm_gate_up", "mm_down", "attention")}
    flop = dict(algo)
    out_layer = max(i for i, s in enumerate(shapes) if s["own_kv"]) if "gather_out" in prof else len(shapes)
    for i, s in enumerate(shapes):
        for k, v in layer_flop(s).items():
            algo[k] += v
            if i < out_layer or (i == out_layer and k == "mm_qkv"):
                flop[k] += v
    kernels = {}
    total_ms = sum(v[1] for v in prof.values())
    for name, (n, ms) in prof.items():
        entry = {"launches_per_step": n // args.steps, "avg_us": round(ms / n * 1e3, 2), "share": round(ms / total_ms, 4)}
        if name in flop:
            tf = flop[name] * args.steps / (ms * 1e-3) / 1e12
            entry.update(tflops=round(tf, 1), mfma_frac=round(tf / PEAK_F16_TFLOPS, 4))
        kernels[name] = entry
    pub = spec["published_ms"]
    out = {
        "metric": "cold latency (Gemma 4 E2B-shaped Q4_0, 12 Qs, 2,000-token state, 2,663 tokens), 1 GPU",
        "value": round(cold_s * 1e3, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(cold_s * 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(cold_s * 1e3 / pub["cold"], 6),
        "dtype": "q4_0 weights, f16 MFMA, f32 accumulate",
        "data": "synthetic (seeded random-init weights and token ids)",
        "config": {"workload": f"{args.config}: Gemma 4 E2B-shaped Q4_0 (35 layers, d 1536, head_dim 256/512, "
                               "20 K/V-sharing layers, per-layer inputs 256), vocab 25k, state 2000 + 12 branches "
                               "(663 tokens), 26 label logits + full-row log-sum-exp readout", "tokens": T, "state_tokens": P, "branches": len(bts)},
        "published_ms": pub,
        "warm_ms": round(warm_s * 1e3, 4),
        "warm_vs_published": round(warm_s * 1e3 / pub["warm"], 6),
        "questions_per_s": round(len(bts) / cold_s, 2),
        "cold_tok_per_s": round(T / cold_s, 1),
        "api_ms": {"cold": round(api_cold_ms, 3), "warm": round(api_warm_ms, 3)},
        "warm_vs_cold_max_abs_logit": warm_equal_cold,
        "pass_tflops": round(sum(flop.values()) / cold_s / 1e12, 2),
        "pass_tflops_algorithmic": round(sum(algo.values()) / cold_s / 1e12, 2),
        "kernels": kernels,
        "load_s": round(load_s, 2),
    }
    print(json.dumps(out))
    return 0


def bench_encoder(args) -> int:
    """the Laya path (mmBERT-base-shaped encoder +
    two decision-head layers, Q8_0) over 64 requests x 3 questions of 256
    tokens in one packed pass; a step is that pass with ids and metadata
    already in HBM."""
    import grande_amd as g
    from grande_amd import laya as ly

    spec = ly.C4
    m = spec["model"]
    cfg = ly.laya_config_json(**m, head_layers=2, act_costs={"ask": 1.0, "escalate": 2.0}, cls=1, sep=2, mask=4,
                              pad=0)
    rng = np.random.default_rng(SEED)
    seqs = encoder_seqs(spec, rng)
    nq, L = len(seqs), spec["seq_len"]
    T = nq * L
    t0 = time.perf_counter()
    weights = ly.synth_weights(cfg, SEED, spec["dtype"], spec["dtype"])
    eng = ly.LayaEngine.new(weights, T, 2 * nq)
    load_s = time.perf_counter() - t0
    t = time.perf_counter()
    outs = eng.evaluate(seqs)
    api_ms = (time.perf_counter() - t) * 1e3

    def timed(steps, warmup):
        eng.prepare(seqs)
        for _ in range(warmup):
            eng.launch()
        eng.sync()
        t = time.perf_counter()
        for _ in range(steps):
            eng.launch()
        eng.sync()
        return (time.perf_counter() - t) / steps

    step_s = timed(args.steps, args.warmup)
    eng.profile(True)
    timed(args.steps, 0)
    prof = eng.profile_report()
    eng.profile(False)

    d, ff, H = m["d"], m["ff"], m["heads"]
    layers = m["layers"]
    n_global = sum(1 for i in range(layers) if i % m["global_every"] == 0)
    pairs_g, pairs_l = encoder_pairs(L, 0) * nq, encoder_pairs(L, m["local_attention"] // 2) * nq
    flops = {"mm_qkv": 2.0 * T * 3 * d * d, "mm_o": 2.0 * T * d * d, "mm_wi": 2.0 * T * 2 * ff * d,
             "mm_wo": 2.0 * T * ff * d, "mm_in": 2.0 * T * 3 * d * d, "mm_out": 2.0 * T * d * d,
             "mm_l1": 2.0 * T * 4 * d * d, "mm_l2": 2.0 * T * 4 * d * d,
             "attention": 4.0 * 64 * H * (n_global * pairs_g + (layers - n_global) * pairs_l) / layers,
             "head_attention": 4.0 * 64 * H * pairs_g}
    kernels = {}
    total_ms = sum(v[1] for v in prof.values())
    for name, (n, ms) in prof.items():
        avg_us = ms / n * 1e3
        entry = {"launches_per_step": n // args.steps, "avg_us": round(avg_us, 2), "share": round(ms / total_ms, 4)}
        if name in flops:
            tf = flops[name] / (avg_us * 1e-6) / 1e12
            entry.update(tflops=round(tf, 1), mfma_frac=round(tf / PEAK_F16_TFLOPS, 4))
        kernels[name] = entry
    dom = max((k for k in kernels if k in flops), key=lambda k: prof[k][1])
    dom_tf = kernels[dom]["tflops"]
    pass_flop = sum(flops[k] * kernels[k]["launches_per_step"] for k in flops if k in kernels)
    out = {
        "metric": "questions/sec (mmBERT-base Laya Q8_0, 64 requests x 3 questions of 256 tokens), 1 GPU",
        "value": round(nq / step_s, 2),
        "unit": "questions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights, f16 MFMA, f32 accumulate",
        "data": "synthetic (seeded random-init weights and token ids)",
        "config": {"workload": "c4: mmBERT-base-shaped encoder (22 layers, d 768, 12 heads, ff 1152, window 64) + "
                               "2 decision-head layers, Q8_0, vocab 56k, 192 sequences x 256 tokens, scorer at "
                               "each [MASK]", "tokens": T, "sequences": nq},
        "tok_per_s": round(T / step_s, 1),
        "api_ms": round(api_ms, 3),
        "pass_tflops": round(pass_flop / step_s / 1e12, 2),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": dom_tf, "peak": PEAK_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(dom_tf / PEAK_F16_TFLOPS, 4),
                     "traffic": profiled_traffic("c4", dom)},
        "kernels": kernels,
        "load_s": round(load_s, 2),
    }
    if not args.no_cpu:
        import oracle

        orc = oracle.Laya(cfg, list(weights.tensors()))
        sample = seqs[:4]
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        t = time.perf_counter()
        rows = orc.hidden([(s.ids, s.markers, s.qtype) for s in sample])
        scores = [orc.score(r) for r in rows]
        cpu_s = time.perf_counter() - t
        worst = max(float(np.max(np.abs(o.logits - sc[0]))) for o, sc in zip(outs, scores))
        out["cpu_baseline"] = {"value": round(len(sample) / cpu_s, 4), "unit": "questions/s", "cores": threads, "cpu_model": cpu_model(),
                               "kind": "port", "sample": f"{len(sample)} of the {nq} questions (256 tokens each, "
                               "22 + 2 layers) + scorer, C restatement with the GPU path's rounding points, OpenMP",
                               "seconds": round(cpu_s, 3), "gpu_speedup": round((nq / step_s) / (len(sample) / cpu_s), 1)}
        out["parity"] = {"max_abs_scorer_logit_diff": worst, "questions_checked": len(sample)}
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
