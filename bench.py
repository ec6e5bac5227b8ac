#!/usr/bin/env python3
"""Benchmark: Qwen3-30B-A3B-shaped Q4_K MoE FFN decode on one MI355X.

Workload: 48 MoE FFN layers (H=2048, E=128, top-8,
F=768), Q4_K gate/up/down experts quantized on the GPU from seeded N(0, 0.02)
fp32, fp32 routers N(0, 0.02), RMSNorm (eps 1e-6) between layers; batch-1
decode, each step a fresh N(0, 1) token input pushed through all 48 layers.
A step = one token through the whole 48-layer stack.

Prints one JSON line: decode tok/s (whole job), the roofline of the dominant
kernel measured with HIP events on its own stream, and the reference ggml CPU
backend (built from the reference's sources) timed on this host's cores on the
same 48 layers and tokens, with the GPU's ids and outputs checked against it.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

H, E, K_USED, F, N_LAYER = 2048, 128, 8, 768, 48
RMS_EPS = 1e-6
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_xcd_q4k_30b_pmc.txt"
KERNEL_NAMES = {1: "k_decode_stack<8,3,Q4_K>", 2: "k_decode_xcd<8,3,4> (XCD-local exchange words)",
                3: "k_decode_xcd<8,3,4> (device-scope exchange words)",
                4: "k_decode_xcd_wide<16,6,4,Q6_K> (XCD-local exchange words)",
                5: "k_decode_xcd_wide<16,6,4,Q6_K> (device-scope exchange words)"}


# The sources of the headline kernel: a counter summary under profiles/ holds
# their SHA-256 beside its bytes, and its traffic is reported only for them.
KERNEL_SOURCES = ["decode_xcd.hip", "qw_xcd.hpp", "qw_decode.hpp", "qw_kernels.hpp", "qw_common.hpp", "qw_sort.hpp"]


def kernel_sources_sha256() -> str:
    import hashlib
    h = hashlib.sha256()
    for name in KERNEL_SOURCES:
        h.update((ROOT / "questwend_amd" / "csrc" / name).read_bytes())
    return h.hexdigest()


def measured_traffic(path: str):
    """(HBM bytes per decode launch, note) from a committed rocprofv3 counter
    summary: the bytes only when the summary's kernel_sources_sha256 matches the
    sources built here, else (None, why)."""
    try:
        lines = Path(path).read_text().splitlines()
    except OSError:
        return None, f"no counter summary at {path}"
    val, sha = None, None
    for line in lines:
        t = line.strip()
        try:
            if t.startswith("hbm_bytes_per_launch"):
                val = int(float(t.split("=", 1)[1].split()[0]))
            elif t.startswith("kernel_sources_sha256"):
                sha = t.split("=", 1)[1].split()[0]
        except (ValueError, IndexError):
            pass
    if val is None:
        return None, "the counter summary holds no hbm_bytes_per_launch"
    if sha != kernel_sources_sha256():
        return None, "the counter summary was measured on other kernel sources (stale); re-measure"
    return val, f"rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by the copy probe ({Path(path).name})"


def algorithmic_bytes_per_token() -> int:
    from questwend_amd import Q4_K, row_size
    expert = 2 * F * row_size(Q4_K, H) + H * row_size(Q4_K, F)        # gate + up + down of one expert
    router = E * H * 4
    return N_LAYER * (K_USED * expert + router)                        # activations are negligible


def make_weights(torch, ops, Q4_K, seed: int):
    """Per layer: router f32 [E, H]; gate/up [E*F, row(H)]; down [E*H, row(F)] (uint8)."""
    from questwend_amd import row_size
    dev = "cuda:0"
    layers = []
    chunk = 16  # experts generated + quantized per step (bounded fp32 scratch)
    tmp = torch.empty(chunk * F * H, dtype=torch.float32, device=dev)
    for l in range(N_LAYER):
        router = torch.empty((E, H), dtype=torch.float32, device=dev)
        ops.randn_(router, seed * 1000 + l * 10 + 0, 0.0, 0.02)
        mats = []
        for role, (rows, cols) in enumerate(((F, H), (F, H), (H, F))):
            q = torch.empty((E * rows, row_size(Q4_K, cols)), dtype=torch.uint8, device=dev)
            for e0 in range(0, E, chunk):
                n = chunk * rows * cols
                ops.randn_(tmp[:n], seed * 1000 + l * 10 + 1 + role * 100000 + e0, 0.0, 0.02)
                ops.quantize_chunk_into(Q4_K, tmp[:n].view(chunk * rows, cols), q[e0 * rows:(e0 + chunk) * rows])
            mats.append(q)
        layers.append((router, *mats))
    torch.cuda.synchronize()
    del tmp
    return layers


def host_cpu() -> dict:
    """CPU model and topology of this host, and the threads this process may use."""
    model, sockets, cores = "unknown", set(), set()
    try:
        phys = None
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name":
                model = val
            elif key == "physical id":
                phys = val
                sockets.add(val)
            elif key == "core id":
                cores.add((phys, val))
    except OSError:
        pass
    n_sock = max(1, len(sockets))
    per_socket = max(1, len(cores) // n_sock) if cores else (os.cpu_count() or 1)
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"model": model, "sockets": n_sock, "cores_per_socket": per_socket, "cpus_available": avail}


def cpu_reference_stack(layers, xs, n_warmup: int, gpu_out, gpu_ids, gpu_layer=None, n_forced: int = 4):
    """BASELINE.md's CPU plan on the decode workload: the reference ggml CPU
    backend (oracle/_ref, built from the reference's own sources) running the
    same 48 layers (weights copied from the GPU) on the same tokens: n_warmup
    warm-up steps, then every timed step, each a token through all 48 layers,
    timed with steady_clock; median and p90 per token.  Threads: the physical
    cores of one socket (capped by the CPUs this process may use).  The timed
    build takes ggml's AVX-512 branch when the host has it.

    Parity, free-running over the same steps: against the AVX2 build (the
    branch the GPU path reproduces) ids and the last layer's output must be
    bit-identical; against the AVX-512 build, the first step/layer where ids
    diverge with the top-k margin there (its float order differs, and a one-ulp
    difference that moves a Q8_K rounding grows from layer to layer).
    Teacher-forced against the AVX-512 build (gpu_layer(l, x) -> (out, ids): the
    GPU's per-layer path, bit-identical to the stack): every layer of n_forced
    steps takes the CPU's own input; ids must agree unless the top-k margin is
    within rounding, and max|gpu - cpu| / max|cpu| of the layer output must
    stay within 1e-3."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_lib import Q4_K, REF_SO, REF_SO_AVX512, LayerWeights, RefGGML, have_ref_avx512
    if not REF_SO.exists():
        return None, None
    cpu = host_cpu()
    n_thr = max(1, min(cpu["cores_per_socket"], cpu["cpus_available"]))
    t0 = time.perf_counter()
    lws = []
    for (router, gate, up, down) in layers:
        lw = LayerWeights.__new__(LayerWeights)
        lw.H, lw.E, lw.k, lw.F = H, E, K_USED, F
        lw.type_gate = lw.type_up = lw.type_down = Q4_K
        lw.router = router.cpu().numpy()
        lw.gate, lw.up, lw.down = (m.cpu().numpy().reshape(-1) for m in (gate, up, down))
        lw.n_slots, lw.slot_of = E, None
        lws.append(lw)
    t_copy = time.perf_counter() - t0
    has512 = have_ref_avx512()
    runs = {}
    for name, path in (("avx2", REF_SO), ("avx512", REF_SO_AVX512 if has512 else None)):
        if path is None:
            continue
        ref = RefGGML(path)
        Ls = [ref.layer(lw, 1, rms_eps=RMS_EPS, n_threads=n_thr) for lw in lws]
        runs[name] = (ref.isa(), ref.stack_run(Ls, xs, n_warmup, n_thr))
        del Ls
    timed = "avx512" if "avx512" in runs else "avx2"
    isa, r = runs[timed]
    st = r["step_s"]
    med, p90 = float(np.median(st)), float(np.percentile(st, 90))
    n_steps = len(st)
    base = {"value": round(1.0 / med, 2), "unit": "tok/s", "cores": n_thr, "kind": "reference",
            "sample": f"all {N_LAYER} layers, {n_warmup} warm-up + {n_steps} timed steps (T=1), same weights and "
                      f"tokens as the GPU run; tok/s = 1 / median per-token time",
            "median_ms_per_token": round(med * 1e3, 3), "p90_ms_per_token": round(p90 * 1e3, 3),
            "isa": "AVX-512" if isa == 512 else "AVX2", "threads": n_thr,
            "cpu": f"{cpu['model']}, {cpu['sockets']} socket(s) x {cpu['cores_per_socket']} cores, "
                   f"{cpu['cpus_available']} CPUs available",
            "weights_to_host_s": round(t_copy, 1)}
    if "avx512" in runs and timed != "avx2":
        a2 = runs["avx2"][1]["step_s"]
        base["avx2_median_ms_per_token"] = round(float(np.median(a2)) * 1e3, 3)
    rel = lambda g, c: float(np.abs(g - c).max() / max(np.abs(c).max(), 1e-30))  # noqa: E731
    a = runs["avx2"][1]
    par = {"metric": "max|gpu-cpu| / max|cpu| of a layer output",
           "avx2_free_running": {
               "steps": n_steps, "layers": N_LAYER,
               "ids_equal_steps": int(sum(np.array_equal(gpu_ids[s], a["ids"][s]) for s in range(n_steps))),
               "out_bits_equal_steps": int(sum(np.array_equal(gpu_out[s].view(np.int32), a["out"][s].view(np.int32))
                                               for s in range(n_steps))),
               "min_topk_margin": float(a["margin"].min())}}
    if "avx512" in runs:
        b = runs["avx512"][1]
        first, agree = None, 0
        for s_ in range(n_steps):
            if np.array_equal(gpu_ids[s_], b["ids"][s_]):
                agree += 1
            elif first is None:
                l = int(np.nonzero((gpu_ids[s_] != b["ids"][s_]).any(axis=1))[0][0])
                first = {"step": s_, "layer": l, "topk_margin": float(b["margin"][s_, l])}
        par["avx512_free_running"] = {"steps": n_steps, "ids_equal_steps": agree, "first_ids_divergence": first}
        if gpu_layer is not None:
            ref = RefGGML(REF_SO_AVX512)
            RL = [ref.layer(lw, 1, rms_eps=RMS_EPS, n_threads=n_thr) for lw in lws]
            n, same, err, worst_margin = 0, 0, 0.0, 0.0
            for s_ in range(min(n_forced, n_steps)):
                x = xs[n_warmup + s_: n_warmup + s_ + 1]
                for l in range(N_LAYER):
                    c = RL[l](x)
                    go, gi = gpu_layer(l, x)
                    n += 1
                    if np.array_equal(gi, c["ids"][0]):
                        same += 1
                    else:
                        p = np.sort(c["probs"][0])[::-1]
                        worst_margin = max(worst_margin, float(p[K_USED - 1] - p[K_USED]))
                    err = max(err, rel(go, c["out"][0]))
                    x = c["xnext"]
            par["avx512_teacher_forced"] = {"layer_evaluations": n, "ids_equal": same,
                                            "largest_margin_where_ids_differ": worst_margin, "out_max_rel_err": err,
                                            "within_1e-3": err <= 1e-3}
            del RL
    return base, par


def zipf_router_scales(E: int = 128, k: int = 8, s: float = 1.1, T: int = 512, cap_frac: float = 0.55,
                       iters: int = 120, n: int = 20000, seed: int = 1234):
    """configs[2]'s skewed gate: per-expert router row scales under which the
    chance that expert i is among a token's top k follows a Zipf(s) rank profile,
    p_i = min(cap, C i^-s) with C such that the k picks per token add up.  With
    a scale-only skew an expert saturates near half of the tokens, so the profile
    is capped at cap_frac of them; far down the tail the fit runs out of
    probability and those experts get almost nothing (a batch of T tokens then
    has row counts from 0 to about 250, the configured "0 to about 300").

    The router rows are random, so a token's logits are independent normals
    scaled row by row; the scales are fitted on n such draws by a fixed-point
    iteration (deterministic, ~1 s).  Top-k ignores a common factor, so the
    scales are returned with the largest at 1: every row stays within the
    configured N(0, 0.02) size and the logits within a few units (no softmax
    underflow to exact ties).  float32 [E]."""
    import numpy as np
    p = np.arange(1, E + 1, dtype=np.float64) ** (-s)
    cap = cap_frac * T
    lo, hi = 0.0, 1e9
    for _ in range(200):                      # C: the capped profile sums to k picks per token
        C = 0.5 * (lo + hi)
        lo, hi = (C, hi) if np.minimum(cap, C * p).sum() < k * T else (lo, C)
    target = np.minimum(cap, C * p) / T
    z = np.random.default_rng(seed).standard_normal((n, E)).astype(np.float32)
    sc = np.ones(E)
    for _ in range(iters):
        top = np.argpartition(-(z * sc.astype(np.float32)), k - 1, axis=1)[:, :k]
        freq = np.bincount(top.ravel(), minlength=E) / n
        sc *= np.clip((target / np.maximum(freq, 1e-6)) ** 0.5, 0.5, 2.0)
        sc /= np.exp(np.log(sc).mean())
    return (sc / sc.max()).astype(np.float32)


def row_count_profile(counts) -> dict:
    """Shape of a batch's per-expert row counts: largest, experts with none, and
    the log-log slope of the sorted counts over ranks 5..100 (a Zipf(s) profile
    gives -s)."""
    import numpy as np
    c = np.sort(np.asarray(counts))[::-1].astype(np.float64)
    r = np.arange(1, c.size + 1)
    m = (r >= 5) & (r <= min(100, c.size)) & (c > 0)
    slope = float(np.polyfit(np.log(r[m]), np.log(c[m]), 1)[0]) if m.sum() > 2 else None
    return {"max_rows": int(c[0]), "experts_with_no_rows": int((c == 0).sum()),
            "loglog_slope_rank5_100": None if slope is None else round(slope, 3)}


def prefill(args) -> int:
    """one Qwen3-30B-A3B-shaped Q4_K MoE FFN layer, a prefill batch
    of T=512 N(0,1) tokens, router rows skewed so expert popularity follows
    Zipf(1.1).  A step = the whole layer (router, grouping, quantization,
    gate/up/down mul_mat_id, SwiGLU, weighted sum, RMSNorm) for the 512 tokens."""
    import numpy as np
    import torch
    from questwend_amd import Q4_K, ops, row_size

    T = args.tokens
    ops.init(0, 512 << 20)
    dev = "cuda:0"
    router = torch.empty((E, H), dtype=torch.float32, device=dev)
    ops.randn_(router, args.seed * 1000 + 1, 0.0, 0.02)
    router *= torch.from_numpy(zipf_router_scales(E, K_USED, 1.1, T)).to(dev)[:, None]
    mats = []
    tmp = torch.empty(16 * F * H, dtype=torch.float32, device=dev)
    for role, (rows, cols) in enumerate(((F, H), (F, H), (H, F))):
        q = torch.empty((E * rows, row_size(Q4_K, cols)), dtype=torch.uint8, device=dev)
        for e0 in range(0, E, 16):
            ops.randn_(tmp[:16 * rows * cols], args.seed * 1000 + 2 + role * 100000 + e0, 0.0, 0.02)
            ops.quantize_chunk_into(Q4_K, tmp[:16 * rows * cols].view(16 * rows, cols), q[e0 * rows:(e0 + 16) * rows])
        mats.append(q)
    del tmp
    L = ops.make_layer(H, E, K_USED, F, router, *mats, (Q4_K,) * 3)
    x = torch.empty((T, H), dtype=torch.float32, device=dev)
    ops.randn_(x, args.seed + 555, 0.0, 1.0)
    torch.cuda.synchronize()

    def timed(min_rows: int, form: int | None = None):
        prev = ops.set_mfma_min_rows(min_rows)
        prev_f = ops.set_mfma_form(form) if form is not None else None
        try:
            for _ in range(args.warmup):
                ops.ffn_layer(L, x, rms_eps=RMS_EPS)
            torch.cuda.synchronize()
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(args.steps)]
            t0 = time.perf_counter()
            for a, b in evs:
                a.record()
                r = ops.ffn_layer(L, x, rms_eps=RMS_EPS)
                b.record()
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
            return wall / args.steps, sum(a.elapsed_time(b) for a, b in evs) / args.steps / 1000.0, r
        finally:
            ops.set_mfma_min_rows(prev)
            if prev_f is not None:
                ops.set_mfma_form(prev_f)

    step_s, ev_s, (out, xn, ids, w) = timed(args.mfma_min_rows)          # the library default: exact
    if args.exact_only:   # (kernel traces of the default form alone)
        auto_s = bs_s = gemv_s = out_a = out_b = out_g = None
    else:
        auto_s, _, (out_a, _, _, _) = timed(args.mfma_min_rows, ops.MFMA_AUTO)
        bs_s, _, (out_b, _, _, _) = timed(args.mfma_min_rows, ops.MFMA_BLOCK_SUM)
        gemv_s, _, (out_g, _, _, _) = timed(0)

    def rel(a):   # vs the GEMV, which (like the exact matrix-core form) replays ggml's float steps
        if a is None:
            return None
        return float(f"{float((a.double() - out_g.double()).abs().max() / out_g.double().abs().max().clamp_min(1e-30)):.3e}")

    def ms(t):
        return None if t is None else round(t * 1e3, 4)

    same = None if out_g is None else bool(torch.equal(out.view(torch.int32), out_g.view(torch.int32)))
    counts = np.bincount(ids.cpu().numpy().reshape(-1), minlength=E)
    expert_bytes = 2 * F * row_size(Q4_K, H) + H * row_size(Q4_K, F)
    wbytes = int((counts > 0).sum()) * expert_bytes + E * H * 4          # unique weights touched + router
    macs = T * K_USED * (2 * F * H + H * F)                               # int8 MACs of the three projections
    cpu = None
    if not args.no_cpu_baseline:
        cpu = prefill_cpu_baseline(host_layer_weights(router, *mats, (Q4_K,) * 3, H, E, K_USED, F), x, T)
    line = {
        "metric": "prefill tok/s + achieved HBM GB/s and int8 MFMA rate, Q4_K MoE FFN layer 30B-A3B",
        "value": round(T / step_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_K x q8_K -> int32 (MFMA i8) -> f32", "data": "synthetic (seeded, router Zipf(1.1)-skewed)",
        "config": {"workload": "Qwen3-30B-A3B MoE FFN layer, prefill T=512 (configs[2])", "n_embd": H,
                   "n_expert": E, "n_expert_used": K_USED, "n_ff_exp": F, "tokens": T, "weights": "Q4_K",
                   "path": f"qwmoe_ffn_layer (mfma_min_rows {args.mfma_min_rows}, the default exact matrix-core "
                           "form: ggml's bits)"},
        "rows_per_expert": {**row_count_profile(counts), "ge32": int((counts >= 32).sum())},
        "roofline": {"bound": "hbm", "achieved": round(wbytes / ev_s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(wbytes / ev_s / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_step": wbytes, "avg_step_ms": round(ev_s * 1e3, 4),
                     "int8_mac_rate_tops": round(macs / ev_s / 1e12, 2),
                     "int8_mac_frac_of_2500_tmacs": round(macs / ev_s / 2.5e15, 4)},
        "exact_mfma_equals_gemv_bitwise": same,
        "auto_form_ms_per_step": ms(auto_s),
        "auto_form_rel_err_vs_gemv": rel(out_a),
        "block_sum_everywhere_ms_per_step": ms(bs_s),
        "block_sum_everywhere_rel_err_vs_gemv": rel(out_b),
        "gemv_only_ms_per_step": ms(gemv_s),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_chain_baseline(host_layers, xs, T: int, n_layer_total: int, budget_s: float = 15.0):
    """The reference ggml CPU backend (oracle/_ref, AVX-512 branch when the host
    has it) running a chain of layers at T tokens: each step pushes T tokens
    through every layer of host_layers (x -> layer -> RMSNorm -> next layer),
    timed per step; one warm-up step, then steps until budget_s of CPU work.
    When host_layers is a sample of the workload's n_layer_total layers, the
    per-step time is scaled by n_layer_total / len(host_layers).  Threads: the
    physical cores of one socket.  None without the reference build."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_lib import REF_SO, REF_SO_AVX512, RefGGML, have_ref_avx512
    if not REF_SO.exists():
        return None
    cpu = host_cpu()
    n_thr = max(1, min(cpu["cores_per_socket"], cpu["cpus_available"]))
    ref = RefGGML(REF_SO_AVX512 if have_ref_avx512() else REF_SO)
    RL = [ref.layer(lw, T, rms_eps=RMS_EPS, n_threads=n_thr) for lw in host_layers]
    times, t_all, i = [], time.perf_counter(), 0
    while True:
        x = np.ascontiguousarray(xs[i % len(xs)][:T], np.float32)
        t0 = time.perf_counter()
        for R in RL:
            x = R(x)["xnext"]
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
        i += 1
        if (time.perf_counter() - t_all > budget_s and len(times) >= 3) or len(times) >= 2000:
            break
    med = float(np.median(times)) * n_layer_total / len(host_layers)
    return {"value": round(T / med, 2), "unit": "tok/s", "cores": n_thr, "kind": "reference",
            "sample": f"{len(times)} steps of T={T} through {len(host_layers)} of the {n_layer_total} layers "
                      f"(per-step time scaled by {n_layer_total}/{len(host_layers)}); tok/s = T / median step",
            "median_ms_per_step": round(med * 1e3, 3), "isa": "AVX-512" if ref.isa() == 512 else "AVX2",
            "threads": n_thr, "cpu": cpu["model"]}


def host_layer_weights(router, gate, up, down, types, H_, E_, k_, F_):
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_lib import LayerWeights
    lw = LayerWeights.__new__(LayerWeights)
    lw.H, lw.E, lw.k, lw.F = H_, E_, k_, F_
    lw.type_gate, lw.type_up, lw.type_down = types
    lw.router = router.cpu().numpy()
    lw.gate, lw.up, lw.down = (m.cpu().numpy().reshape(-1) for m in (gate, up, down))
    lw.n_slots, lw.slot_of = E_, None
    return lw


def prefill_cpu_baseline(lw, x, T: int):
    """The reference ggml CPU backend (oracle/_ref) on the same layer (host
    weights lw) and batch: evaluations of the T-token graph for about 10 s on
    the physical cores of one socket."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_lib import REF_SO, RefGGML
    if not REF_SO.exists():
        return None
    cpu = host_cpu()
    n_thr = max(1, min(cpu["cores_per_socket"], cpu["cpus_available"]))
    run = RefGGML().layer(lw, T, rms_eps=RMS_EPS, n_threads=n_thr)
    xh = x.cpu().numpy()
    run(xh, n_threads=n_thr)
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < 10.0 or reps == 0:
        run(xh, n_threads=n_thr)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    return {"value": round(T / dt, 2), "unit": "tok/s", "cores": n_thr, "kind": "reference",
            "sample": f"{reps} evaluations of the T={T} layer graph in {dt * reps:.1f}s", "ms_per_layer": round(dt * 1e3, 3)}


def verify_cpu_protocol(lw, T: int, n_steps: int, rho: float, seed: int):
    """configs[3]'s protocol on the reference ggml CPU backend: n_steps seeded
    batches of T tokens, N(0,1) correlated at rho, through one layer (lw); each
    step timed with perf_counter; median and p90 per step."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_lib import REF_SO, REF_SO_AVX512, RefGGML, have_ref_avx512
    if not REF_SO.exists():
        return None
    cpu = host_cpu()
    n_thr = max(1, min(cpu["cores_per_socket"], cpu["cpus_available"]))
    ref = RefGGML(REF_SO_AVX512 if have_ref_avx512() else REF_SO)
    run = ref.layer(lw, T, rms_eps=RMS_EPS, n_threads=n_thr)
    rng = np.random.default_rng(seed)
    times = []
    for i in range(n_steps + 8):
        c = rng.standard_normal(lw.H)
        x = (np.sqrt(rho) * c + np.sqrt(1.0 - rho) * rng.standard_normal((T, lw.H))).astype(np.float32)
        t0 = time.perf_counter()
        run(x)
        if i >= 8:
            times.append(time.perf_counter() - t0)
    med, p90 = float(np.median(times)), float(np.percentile(times, 90))
    return {"median_ms_per_layer": round(med * 1e3, 4), "p90_ms_per_layer": round(p90 * 1e3, 4), "cores": n_thr,
            "isa": "AVX-512" if ref.isa() == 512 else "AVX2", "steps": n_steps, "T": T}


def expert_cache_bench(args) -> int:
    """The configs[1] decode stack (48 Q4_K layers of the 30B-A3B shape) with
    its experts in pinned host memory and a fraction ``--resident`` of them in
    HBM slot pools fed by qwmoe_expert_cache (the RAM tier of
    core/expert_cache.cpp:355-364).  A step = one token: the whole-stack kernel
    speculating on the resident set, the ids it used checked against the
    residency (qwmoe_expert_cache_verify), and on a miss the per-layer path
    (router -> ensure -> layer, core/runtime.cpp:2458-2662).  Router rows are
    Zipf(--zipf)-skewed (0: unskewed).  Every timed token's output is compared
    bitwise with the all-resident stack afterwards."""
    import numpy as np
    import torch
    from questwend_amd import Q4_K, ops, row_size

    ops.init(0, 256 << 20)
    dev = "cuda:0"
    layers = make_weights(torch, ops, Q4_K, args.seed)
    if args.zipf > 0:
        sc = torch.from_numpy(zipf_router_scales(E, K_USED, args.zipf)).to(dev)[:, None]
        for lay in layers:
            lay[0].mul_(sc)
    # the RAM tier: every expert tensor in pinned host memory
    host = [[None] * N_LAYER for _ in range(3)]
    for l, lay in enumerate(layers):
        for r in range(3):
            m = lay[1 + r]
            h = torch.empty(m.numel(), dtype=torch.uint8, pin_memory=True)
            h.copy_(m.view(-1))
            host[r][l] = h
    torch.cuda.synchronize()
    # plain H2D probe: one 1 GiB pinned -> device copy
    probe_h = torch.empty(1 << 30, dtype=torch.uint8, pin_memory=True)
    probe_d = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    probe_d.copy_(probe_h, non_blocking=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        probe_d.copy_(probe_h, non_blocking=True)
    torch.cuda.synchronize()
    h2d_probe = 3 * (1 << 30) / (time.perf_counter() - t0) / 1e9
    del probe_h, probe_d

    shapes = ((H, F), (H, F), (F, H))
    slab = [row_size(Q4_K, shapes[r][0]) * shapes[r][1] for r in range(3)]
    total = sum(slab) * E * N_LAYER
    budget = int(total * args.resident)
    srcs = [[{"type": Q4_K, "ne0": shapes[r][0], "ne1": shapes[r][1], "host": host[r][l].data_ptr()}
             for l in range(N_LAYER)] for r in range(3)]
    cache = ops.ExpertCache(N_LAYER, E, srcs, budget, K_USED, copy_engine=args.copy_engine)
    resident = [ops.make_layer(H, E, K_USED, F, r, g, u, d, (Q4_K,) * 3) for (r, g, u, d) in layers]
    cached = []
    for l, (r, g, u, d) in enumerate(layers):
        L = ops.make_layer(H, E, K_USED, F, r, g, u, d, (Q4_K,) * 3)
        cache.layer(l, L)
        cached.append(L)
    spec = ops.DecodeStack(cached, RMS_EPS, keepalive=(layers, host))
    n_per_layer = min(E, cache.capacity(0) // N_LAYER)

    # cold fill: the first n_per_layer experts of every layer (the Zipf-hot ones)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for l in range(N_LAYER):
        cache.ensure(l, list(range(n_per_layer)))
    cache.sync()
    fill_s = time.perf_counter() - t0
    fill_bytes = cache.stats()["fetch_bytes"]

    n_steps = args.steps + args.warmup
    xs = torch.empty((n_steps, H), dtype=torch.float32, device=dev)
    ops.randn_(xs, args.seed + 777, 0.0, 1.0)
    outs = torch.empty((n_steps, H), dtype=torch.float32, device=dev)
    def step(i):
        x = xs[i]
        out, _, ids, _ = spec(x)
        if cache.verify(ids.cpu()) == 0:          # accepted (touches every used expert)
            outs[i].copy_(out)
            return True
        xl = x.view(1, H)
        for l in range(N_LAYER):                    # decode_cached: router, ids back, ensure, layer
            o, xl, _, _ = cache.run_layer(l, cached[l], xl, rms_eps=RMS_EPS)
        outs[i].copy_(o.view(-1))
        return False

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    st0 = cache.stats()
    t0 = time.perf_counter()
    accepted = sum(step(args.warmup + i) for i in range(args.steps))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    st1 = cache.stats()

    # the same tokens through the all-resident stack
    ref = ops.DecodeStack(resident, RMS_EPS, keepalive=layers)
    same = True
    for i in range(args.warmup, n_steps):
        o, _, _, _ = ref(xs[i], want_ids=False)
        same &= bool(torch.equal(o.view(torch.int32), outs[i].view(torch.int32)))
    torch.cuda.synchronize()
    fetched = st1["fetch_bytes"] - st0["fetch_bytes"]
    miss = st1["misses"] - st0["misses"]
    line = {
        "metric": "offloaded decode tok/s, 30B-A3B Q4_K MoE FFN stack, experts in pinned host memory, "
                  f"{args.resident:.0%} of them in HBM slot pools",
        "value": round(args.steps / wall, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall * 1e3 / args.steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_K x q8_K -> f32",
        "data": f"synthetic (seeded; router rows Zipf({args.zipf})-skewed)" if args.zipf > 0 else "synthetic (seeded)",
        "config": {"workload": "configs[1] decode stack through the expert cache (RAM tier)", "n_layer": N_LAYER,
                   "n_embd": H, "n_expert": E, "n_expert_used": K_USED, "n_ff_exp": F, "weights": "Q4_K",
                   "resident_fraction": args.resident, "pool_slots": [p["n_slots"] for p in cache.pools()],
                   "zipf": args.zipf, "scattered_fetch": "copy engine" if args.copy_engine else "gather kernel"},
        "accepted_speculative": accepted, "repaired_per_layer": args.steps - accepted,
        "misses_per_token": round(miss / args.steps, 2), "fetched_mb_per_token": round(fetched / args.steps / 1e6, 2),
        "fetch_gbps_during_run": round(fetched / wall / 1e9, 2),
        "cold_fill": {"bytes": fill_bytes, "seconds": round(fill_s, 4), "gbps": round(fill_bytes / fill_s / 1e9, 2)},
        "h2d_probe_gbps": round(h2d_probe, 2),
        "roofline": {"bound": "pcie", "achieved": round(fill_bytes / fill_s / 1e9, 2), "peak": 64.0, "unit": "GB/s",
                     "frac": round(fill_bytes / fill_s / 1e9 / 64.0, 4), "traffic": None,
                     "note": "cold fill of the pools through ensure(); peak = PCIe 5.0 x16 per direction"},
        "matches_all_resident_bitwise": same,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    spec.close()
    ref.close()
    cache.close()
    return 0


def verify_bench(args) -> int:
    """the verify batch of speculative decoding, T = n_draft + 1
    tokens (1..--tokens) per step through the configs[1] stack (48 Q4_K layers of
    the 30B-A3B shape), the T tokens' activations N(0,1) correlated at rho = 0.8
    so that their experts partly overlap.  qwmoe_layer_stack runs 2 <= T <= 8 as
    one persistent launch (verify_xcd.hip) where the device allows; beside it the
    per-layer chain (the same stack created with QWMOE_VERIFY_XCD=0: one captured
    graph of five launches per layer, bitwise compared) and the T tokens decoded
    one launch each by the persistent decode stack."""
    import numpy as np
    import torch
    from questwend_amd import Q4_K, ops, row_size

    ops.init(0, 256 << 20)
    layers = make_weights(torch, ops, Q4_K, args.seed)
    Ls = [ops.make_layer(H, E, K_USED, F, r, g, u, d, (Q4_K,) * 3) for (r, g, u, d) in layers]
    Tmax = max(1, args.tokens)
    stack = ops.LayerStack(Ls, RMS_EPS, max_tokens=Tmax, keepalive=layers)
    old = os.environ.get("QWMOE_VERIFY_XCD")
    os.environ["QWMOE_VERIFY_XCD"] = "0"
    try:
        chain = ops.LayerStack(Ls, RMS_EPS, max_tokens=Tmax, keepalive=layers)
    finally:
        if old is None:
            os.environ.pop("QWMOE_VERIFY_XCD")
        else:
            os.environ["QWMOE_VERIFY_XCD"] = old
    dstack = ops.DecodeStack(Ls, RMS_EPS, keepalive=layers)
    n = args.steps + args.warmup
    c = torch.empty((n, 1, H), dtype=torch.float32, device="cuda:0")
    z = torch.empty((n, Tmax, H), dtype=torch.float32, device="cuda:0")
    ops.randn_(c, args.seed + 998, 0.0, 1.0)
    ops.randn_(z, args.seed + 999, 0.0, 1.0)
    xs = (c * math.sqrt(0.8) + z * math.sqrt(0.2)).contiguous()
    expert = 2 * F * row_size(Q4_K, H) + H * row_size(Q4_K, F)

    def timed(fn, T, events=False):
        for i in range(args.warmup):
            fn(xs[i, :T])
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        t0 = time.perf_counter()
        for i in range(args.steps):
            if events:
                evs[i][0].record()
            fn(xs[args.warmup + i, :T])
            if events:
                evs[i][1].record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
        return wall, (sum(a_.elapsed_time(b_) for a_, b_ in evs) / args.steps / 1e3 if events else None)

    def dec(x):
        for t in range(x.shape[0]):
            dstack(x[t], want_ids=False)

    rows, same = [], True
    for T in range(1, Tmax + 1):
        g_s, k_s = timed(lambda x: stack(x, want_ids=False), T, events=True)
        c_s, _ = timed(lambda x: chain(x, want_ids=False), T)
        d_s, _ = timed(dec, T)
        uniq = 0
        for i in range(min(4, n)):
            o, xo, ids, w = stack(xs[i, :T])
            o2, xo2, ids2, w2 = chain(xs[i, :T])
            torch.cuda.synchronize()
            same &= bool(torch.equal(ids, ids2)) and all(
                torch.equal(u.view(torch.int32), v.view(torch.int32)) for u, v in ((o, o2), (xo, xo2), (w, w2)))
            uniq += sum(len(np.unique(ids[l].cpu().numpy())) for l in range(N_LAYER))
        uniq /= min(4, n)
        wbytes = uniq * expert + N_LAYER * E * H * 4
        rows.append({"T": T, "ms": round(g_s * 1e3, 3), "avg_launch_ms": round(k_s * 1e3, 4),
                     "per_layer_chain_ms": round(c_s * 1e3, 3),
                     "decode_stack_x_T_ms": round(d_s * 1e3, 3), "verify_tok_s": round(T / g_s, 1),
                     "unique_experts_per_layer": round(uniq / N_LAYER, 2),
                     "weight_gbps": round(wbytes / k_s / 1e9, 1), "weight_bytes_per_step": int(wbytes)})
    last = rows[-1]
    cpu = None
    if not args.no_cpu_baseline:
        # 1000 seeded T-token batches through one layer, on the reference
        # CPU backend; the line's tok/s for the 48-layer stack from its median
        proto = verify_cpu_protocol(host_layer_weights(*layers[0], (Q4_K,) * 3, H, E, K_USED, F), Tmax, 1000, 0.8,
                                    args.seed)
        if proto:
            med = proto["median_ms_per_layer"] * N_LAYER / 1e3
            cpu = {"value": round(Tmax / med, 2), "unit": "tok/s", "cores": proto["cores"], "kind": "reference",
                   "sample": f"configs[3]: 1000 seeded batches of T={Tmax} correlated tokens (rho 0.8) through one "
                             f"layer, 8 warm-up; tok/s = T / ({N_LAYER} x median layer time)",
                   "protocol": proto}
    kname = {1: "the per-layer chain (captured graph)", 2: "k_verify_xcd<8,3,4> (XCD-local exchange words)",
             3: "k_verify_xcd<8,3,4> (device-scope exchange words)"}.get(stack.kernel(), "?")
    line = {
        "metric": "verify-batch tok/s, 30B-A3B Q4_K MoE FFN stack (speculative-decoding verify forward, FFN half)",
        "value": last["verify_tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": last["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_K x q8_K -> f32", "data": "synthetic (seeded; tokens N(0,1) correlated at rho = 0.8)",
        "config": {"workload": "configs[3]: T tokens per step through the configs[1] stack (qwmoe_layer_stack)",
                   "n_layer": N_LAYER, "n_embd": H, "n_expert": E, "n_expert_used": K_USED, "n_ff_exp": F,
                   "weights": "Q4_K", "tokens": Tmax, "path_T_ge_2": kname},
        "per_T": rows,
        "equals_per_layer_chain_bitwise": same,
        "roofline": {"bound": "hbm", "achieved": last["weight_gbps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(last["weight_gbps"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": last["weight_bytes_per_step"], "avg_launch_ms": last["avg_launch_ms"],
                     "kernel": kname,
                     "note": "the batch's distinct experts' weights + routers per step / average launch time (HIP events)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    stack.close()
    chain.close()
    dstack.close()
    return 0


def config5_bench(args) -> int:
    """the large-expert regime, 94 MoE layers (H=4096, E=128, top-8,
    F=1536), Q4_K gate/up and Q6_K down, every layer's experts stored at a seeded
    random slot permutation read through the slot rows.  Decode at batch 1
    through all 94 layers (the persistent decode kernel's wide XCD form, one
    launch per token; the layer stack at T = 1 timed beside it) and prefill of
    1024 tokens through one layer (qwmoe_ffn_layer, Zipf(1.1)-skewed router)."""
    import numpy as np
    import torch
    from questwend_amd import Q4_K, Q6_K, ops, row_size

    H5, E5, K5, F5 = 4096, 128, 8, 1536
    NL5 = args.c5_layers   # 94; fewer only to profile the prefill kernels
    types = (Q4_K, Q4_K, Q6_K)
    ops.init(0, 1 << 30)
    dev = "cuda:0"
    chunk = 8
    tmp = torch.empty(chunk * F5 * H5, dtype=torch.float32, device=dev)
    layers, keep = [], []
    t_gen = time.perf_counter()
    g = torch.Generator().manual_seed(args.seed)
    for l in range(NL5):
        router = torch.empty((E5, H5), dtype=torch.float32, device=dev)
        ops.randn_(router, args.seed * 1000 + l * 10, 0.0, 0.02)
        mats, slots = [], []
        for role, (rows, cols) in enumerate(((F5, H5), (F5, H5), (H5, F5))):
            q = torch.empty((E5 * rows, row_size(types[role], cols)), dtype=torch.uint8, device=dev)
            perm = torch.randperm(E5, generator=g).to(torch.int32)
            for e0 in range(0, E5, chunk):
                n = chunk * rows * cols
                ops.randn_(tmp[:n], args.seed * 1000 + l * 10 + 1 + role * 100000 + e0, 0.0, 0.02)
                # logical experts e0..e0+chunk go to their slots perm[e]
                qc = ops.quantize_chunk(types[role], tmp[:n].view(chunk * rows, cols)).view(chunk, rows, -1)
                q.view(E5, rows, -1)[perm[e0:e0 + chunk].long().to(dev)] = qc
            mats.append(q)
            slots.append(perm.to(dev))
        L = ops.make_layer(H5, E5, K5, F5, router, *mats, types, n_slots=(E5, E5, E5), slots=tuple(slots))
        layers.append(L)
        keep.append((router, mats, slots))
    torch.cuda.synchronize()
    del tmp
    t_gen = time.perf_counter() - t_gen

    # decode: one token through all 94 layers per step, on the persistent decode
    # kernel (its wide XCD form: one launch per token) and, beside it, on the
    # layer stack at T = 1 (five launches per layer, one captured graph)
    dstack = ops.DecodeStack(layers, RMS_EPS, keepalive=keep)
    os.environ["QWMOE_VERIFY_XCD"] = "0"   # the chain (by default the layer stack hands T = 1 to the decode kernel)
    try:
        stack = ops.LayerStack(layers, RMS_EPS, max_tokens=1, keepalive=keep)
    finally:
        os.environ.pop("QWMOE_VERIFY_XCD", None)
    xs = torch.empty((args.steps + args.warmup, 1, H5), dtype=torch.float32, device=dev)
    ops.randn_(xs, args.seed + 4242, 0.0, 1.0)
    # the two paths on the first 8 tokens: ids, weights and outputs bitwise
    same = True
    for i in range(min(8, args.steps + args.warmup)):
        a_ = dstack(xs[i].view(-1))
        b_ = stack(xs[i])
        same = same and torch.equal(a_[2].view(-1), b_[2].reshape(-1)) and all(
            torch.equal(u.reshape(-1).view(torch.int32), v.reshape(-1).view(torch.int32))
            for u, v in ((a_[0], b_[0]), (a_[1], b_[1]), (a_[3], b_[3])))
    dout = torch.empty(H5, dtype=torch.float32, device=dev)
    dxo = torch.empty(H5, dtype=torch.float32, device=dev)
    for i in range(args.warmup):
        dstack.run(xs[i].view(-1), dout, dxo)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        evs[i][0].record()
        dstack.run(xs[args.warmup + i].view(-1), dout, dxo)
        evs[i][1].record()
    torch.cuda.synchronize()
    dec_s = (time.perf_counter() - t0) / args.steps
    kern_ms = sum(a_.elapsed_time(b_) for a_, b_ in evs) / args.steps
    dstatus = dstack.status()
    for i in range(args.warmup):
        stack(xs[i], want_ids=False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        stack(xs[args.warmup + i], want_ids=False)
    torch.cuda.synchronize()
    ls_s = (time.perf_counter() - t0) / args.steps
    expert5 = 2 * F5 * row_size(Q4_K, H5) + H5 * row_size(Q6_K, F5)
    dec_bytes = NL5 * (K5 * expert5 + E5 * H5 * 4)

    # prefill: 1024 tokens through layer 0, router rows Zipf(1.1)-skewed
    L0 = layers[0]
    T5 = 1024
    keep[0][0].mul_(torch.from_numpy(zipf_router_scales(E5, K5, 1.1, T5)).to(dev)[:, None])
    x = torch.empty((T5, H5), dtype=torch.float32, device=dev)
    ops.randn_(x, args.seed + 99, 0.0, 1.0)
    reps = max(3, args.steps // 4)

    def prefill_s(form):
        prev = ops.set_mfma_form(form)
        prev_rows = ops.set_mfma_min_rows(args.mfma_min_rows)   # as the configs[2] prefill line
        try:
            for _ in range(2):
                ops.ffn_layer(L0, x, rms_eps=RMS_EPS)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                r = ops.ffn_layer(L0, x, rms_eps=RMS_EPS)
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) / reps, r
        finally:
            ops.set_mfma_form(prev)
            ops.set_mfma_min_rows(prev_rows)

    pre_s, (out_x, _, ids, _) = prefill_s(ops.MFMA_EXACT)          # the library default
    if args.exact_only:   # (kernel traces of the default form alone)
        pre_auto_s = pre_bs_s = pre_rel = pre_rel_bs = None
    else:
        pre_auto_s, (out, _, _, _) = prefill_s(ops.MFMA_AUTO)
        pre_bs_s, (out_b, _, _, _) = prefill_s(ops.MFMA_BLOCK_SUM)
        pre_rel = float((out.double() - out_x.double()).abs().max() / out_x.double().abs().max().clamp_min(1e-30))
        pre_rel_bs = float((out_b.double() - out_x.double()).abs().max() / out_x.double().abs().max().clamp_min(1e-30))
    counts5 = np.bincount(ids.cpu().numpy().reshape(-1), minlength=E5)
    used = int((counts5 > 0).sum())
    cpu = pre_cpu = None
    if not args.no_cpu_baseline:
        # decode on the CPU: a sample of 24 of the 94 layers, 1..24 (logical expert
        # order: the slot permutation undone; 37 GB of host memory), their per-token
        # time scaled to 94.  (Layer 0's router now carries the prefill's Zipf skew.)
        def host_logical(l):
            router_l, mats_l, slots_l = keep[l]
            logical = [m.view(E5, -1)[sl.long()] for m, sl in zip(mats_l, slots_l)]
            return host_layer_weights(router_l, *logical, types, H5, E5, K5, F5)
        lws = [host_logical(l) for l in range(1, min(25, NL5))] if NL5 > 1 else [host_logical(0)]
        cpu = cpu_chain_baseline(lws, xs[:16].view(-1, 1, H5).cpu().numpy(), 1, NL5)
        del lws
        pre_cpu = prefill_cpu_baseline(host_logical(0), x, T5)   # layer 0 (Zipf router) at T = 1024
    pre_bytes = used * expert5 + E5 * H5 * 4
    pre_macs = T5 * K5 * (2 * F5 * H5 + H5 * F5)
    line = {
        "metric": "configs[4] decode tok/s (94-layer stack, batch 1) and prefill tok/s (T=1024, one layer)",
        "value": round(1.0 / dec_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dec_s * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_K/q6_K x q8_K -> f32", "data": "synthetic (seeded; slot permutation seeded; prefill router Zipf(1.1))",
        "config": {"workload": f"configs[4]: {NL5} layers H=4096 E=128 k=8 F=1536, Q4_K gate/up, Q6_K down, permuted slots",
                   "decode_path": "qwmoe_decode_stack_run: " + KERNEL_NAMES.get(dstack.kernel(), "?") +
                                  f", one launch per token through {NL5} layers",
                   "prefill_path": f"qwmoe_ffn_layer T=1024 (mfma_min_rows {args.mfma_min_rows})"},
        "decode": {"tok_s": round(1.0 / dec_s, 2), "ms_per_token": round(dec_s * 1e3, 3),
                   "avg_launch_ms": round(kern_ms, 4),
                   "weight_bytes_per_token": dec_bytes, "gbps": round(dec_bytes / dec_s / 1e9, 1),
                   "frac_of_8tbs": round(dec_bytes / dec_s / 1e9 / HBM_PEAK_GBS, 4),
                   "device_status": dstatus,
                   "layer_stack_t1_tok_s": round(1.0 / ls_s, 2),
                   "equals_layer_stack_bitwise_8_tokens": bool(same)},
        "prefill": {"tokens": T5, "ms_per_layer": round(pre_s * 1e3, 3), "tok_s": round(T5 / pre_s, 1),
                    "used_experts": used, "rows_per_expert": row_count_profile(counts5),
                    "form": "exact (the library default: ggml's bits)",
                    "auto_form_ms_per_layer": None if pre_auto_s is None else round(pre_auto_s * 1e3, 3),
                    "auto_form_rel_err_vs_exact": None if pre_rel is None else float(f"{pre_rel:.3e}"),
                    "block_sum_form_ms_per_layer": None if pre_bs_s is None else round(pre_bs_s * 1e3, 3),
                    "block_sum_form_rel_err_vs_exact": None if pre_rel_bs is None else float(f"{pre_rel_bs:.3e}"),
                    "roofline": {"bound": "hbm", "achieved": round(pre_bytes / pre_s / 1e9, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(pre_bytes / pre_s / 1e9 / HBM_PEAK_GBS, 4),
                                 "traffic": None, "bytes_per_layer": pre_bytes,
                                 "int8_mac_rate_tops": round(pre_macs / pre_s / 1e12, 2),
                                 "int8_mac_frac_of_2500_tmacs": round(pre_macs / pre_s / 2.5e15, 4),
                                 "note": "used experts' weights + router once per layer / wall time per layer; "
                                         "MACs of the three projections (int8 MFMA peak 5.0 POP/s = 2.5 P MAC/s)"},
                    "cpu_baseline": pre_cpu},
        "roofline": {"bound": "hbm", "achieved": round(dec_bytes / kern_ms / 1e6, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dec_bytes / kern_ms / 1e6 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": KERNEL_NAMES.get(dstack.kernel(), "?") + f" (one launch = one token through {NL5} layers)",
                     "bytes_per_launch": dec_bytes, "avg_launch_ms": round(kern_ms, 4),
                     "note": "selected experts' weights + routers per token / average launch time (HIP events)"},
        "weight_gen_s": round(t_gen, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    stack.close()
    dstack.close()
    return 0


def copy_probe(mib: int = 1024, reps: int = 4) -> int:
    """A plain device copy of known size (torch's copy kernel): run under
    ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` it gives the factor between
    those counters and the bytes a kernel actually moves."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "reps": reps}), flush=True)
    return 0


def graph_replay_ms(fn_, n: int):
    """fn_ captured into one HIP graph (torch's stream capture: the library's
    calls enqueue on the capturing stream and allocate nothing) and replayed n
    times: (ms per replay, the captured call's outputs), or (None, None) when
    capture fails."""
    import torch
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn_()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs = fn_()
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            g.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e3, (g, outs)
    except Exception:  # noqa: BLE001 -- capture is reported as unavailable
        return None, None


def attn_bench(args) -> int:
    """The attention half of Seg A (qwmoe_attn_seg, core/runtime.cpp:1976-2030) and
    a whole decoder layer (qwmoe_decoder_layer) at the Qwen3-30B-A3B attention
    shape: H = 2048, 32 query / 4 kv heads of D = 128, Q4_K q/k/o and Q6_K v
    (seeded synthetic weights quantized on the GPU), f16 KV cache of n_ctx = 4096
    rows.  Timed: decode (T = 1) at n_past = 4095 -- the line's value, tokens per
    second of the attention segment -- a prefill chunk of 512 tokens at n_past 0
    and at n_past 3584, and one decoder layer (attention + the 30B MoE FFN) at
    decode.  roofline: the weight rows and KV-cache rows one decode call reads,
    over its time (HIP events).  cpu_baseline: ggml's own graph for the same
    segment (oracle/_ref, AVX-512 build where the host has it) on the same
    weights and cache at decode."""
    import numpy as np
    import torch
    from questwend_amd import Q4_K, Q6_K, ops, row_size

    NH, NKV, D, N_CTX = 32, 4, 128, 4096
    NQ, NK = NH * D, NKV * D
    types = (Q4_K, Q4_K, Q6_K, Q4_K)
    dev = "cuda:0"
    ops.init(0, 512 << 20)

    def qmat(rows, cols, t, seed):
        f = torch.empty((rows, cols), dtype=torch.float32, device=dev)
        ops.randn_(f, seed, 0.0, 0.02)
        return ops.quantize_chunk(t, f)

    def vec(n, seed, mean=1.0, std=0.1):
        v = torch.empty(n, dtype=torch.float32, device=dev)
        return ops.randn_(v, seed, mean, std)

    sd = args.seed * 1000 + 900
    wq, wk = qmat(NQ, H, types[0], sd + 1), qmat(NK, H, types[1], sd + 2)
    wv, wo = qmat(NK, H, types[2], sd + 3), qmat(H, NQ, types[3], sd + 4)
    an, fn, qn, kn = vec(H, sd + 5), vec(H, sd + 6), vec(D, sd + 7), vec(D, sd + 8)
    kc = torch.empty((N_CTX, NK), dtype=torch.float32, device=dev)
    vc = torch.empty((N_CTX, NK), dtype=torch.float32, device=dev)
    ops.randn_(kc, sd + 9, 0.0, 0.5)
    ops.randn_(vc, sd + 10, 0.0, 0.5)
    kc, vc = kc.half(), vc.half()
    AL = ops.make_attn_layer(H, NH, NKV, D, an, wq, wk, wv, wo, types, qn, kn, fn, kc, vc)
    # the MoE FFN of the decoder layer: one 30B layer (as the decode stack's)
    router = torch.empty((E, H), dtype=torch.float32, device=dev)
    ops.randn_(router, sd + 11, 0.0, 0.02)
    mats = [qmat(E * F, H, Q4_K, sd + 12), qmat(E * F, H, Q4_K, sd + 13), qmat(E * H, F, Q4_K, sd + 14)]
    ML = ops.make_layer(H, E, K_USED, F, router, *mats, (Q4_K,) * 3)
    torch.cuda.synchronize()

    def timed(fn_, n):
        for _ in range(max(2, args.warmup)):
            fn_()
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        t0 = time.perf_counter()
        for a, b in evs:
            a.record()
            fn_()
            b.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / n
        return wall, sum(a.elapsed_time(b) for a, b in evs) / n / 1000.0

    h1 = torch.empty((1, H), dtype=torch.float32, device=dev)
    ops.randn_(h1, sd + 20, 0.0, 1.0)
    hp = torch.empty((512, H), dtype=torch.float32, device=dev)
    ops.randn_(hp, sd + 21, 0.0, 1.0)
    n_past = N_CTX - 1
    dec_wall, dec_ev = timed(lambda: ops.attn_seg(AL, h1, n_past), args.steps)
    pre0_wall, pre0_ev = timed(lambda: ops.attn_seg(AL, hp, 0), max(4, args.steps // 16))
    pre1_wall, pre1_ev = timed(lambda: ops.attn_seg(AL, hp, N_CTX - 512), max(4, args.steps // 16))
    lay_wall, lay_ev = timed(lambda: ops.decoder_layer(AL, ML, h1, n_past), args.steps)
    # the decode call captured into a HIP graph: the same kernels without the
    # host's per-launch cost; the replay's outputs checked against an eager call
    g_ms, g_hold = graph_replay_ms(lambda: ops.attn_seg(AL, h1, n_past), args.steps)
    g_equal = None
    if g_hold is not None:
        g_hold[0].replay()
        torch.cuda.synchronize()
        e_out = ops.attn_seg(AL, h1, n_past)
        torch.cuda.synchronize()
        g_equal = bool(torch.equal(g_hold[1][0], e_out[0]) and torch.equal(g_hold[1][1], e_out[1]))
    status = ops.device_status(clear=True)

    wbytes = NQ * row_size(types[0], H) + NK * row_size(types[1], H) + NK * row_size(types[2], H) + \
        H * row_size(types[3], NQ)
    kvbytes = 2 * (n_past + 1) * NK * 2
    abytes = wbytes + kvbytes + (3 * H + 2 * D) * 4
    moe_bytes = algorithmic_bytes_per_token() // N_LAYER
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(ROOT / "tests"))
        from oracle_lib import REF_SO, REF_SO_AVX512, AttnWeights, RefGGML, have_ref_avx512
        if REF_SO.exists():
            aw = AttnWeights.__new__(AttnWeights)
            aw.H, aw.n_head, aw.n_head_kv, aw.D, aw.types, aw.freq_base = H, NH, NKV, D, types, 1e6
            aw.wq, aw.wk, aw.wv, aw.wo = (t.cpu().numpy().reshape(-1) for t in (wq, wk, wv, wo))
            aw.attn_norm, aw.ffn_norm, aw.q_norm, aw.k_norm = (t.cpu().numpy() for t in (an, fn, qn, kn))
            kch = kc.cpu().numpy().view(np.uint16).copy()
            vch = vc.cpu().numpy().view(np.uint16).copy()
            x = h1.cpu().numpy()
            cpuinfo = host_cpu()
            n_thr = max(1, min(cpuinfo["cores_per_socket"], cpuinfo["cpus_available"]))
            ref = RefGGML(REF_SO_AVX512 if have_ref_avx512() else REF_SO)
            ref.attn_seg(aw, x, n_past, kch, vch, n_threads=n_thr)
            times, t_all = [], time.perf_counter()
            while (time.perf_counter() - t_all < 10.0 or len(times) < 5) and len(times) < 5000:
                t0 = time.perf_counter()
                ref.attn_seg(aw, x, n_past, kch, vch, n_threads=n_thr)
                times.append(time.perf_counter() - t0)
            med = float(np.median(times))
            cpu = {"value": round(1.0 / med, 1), "unit": "tok/s", "cores": n_thr, "kind": "reference",
                   "sample": f"{len(times)} decode steps (T=1 at n_past {n_past}) of ggml's attention graph in "
                             f"{time.perf_counter() - t_all:.1f}s",
                   "median_ms_per_step": round(med * 1e3, 4), "isa": "AVX-512" if ref.isa() == 512 else "AVX2",
                   "threads": n_thr, "cpu": cpuinfo["model"]}
    line = {
        "metric": "attention decode tok/s + achieved HBM GB/s, Qwen3-30B-A3B attention at 4096 context",
        "value": round(1.0 / dec_wall, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dec_wall * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_K/q6_K x q8_K -> f32; f16 KV cache",
        "data": "synthetic (seeded N(0,0.02) weights quantized on the GPU; N(0,0.5) f16 cache; N(0,1) inputs)",
        "config": {"workload": "Qwen3-30B-A3B attention half of Seg A (qwmoe_attn_seg)", "n_embd": H,
                   "n_head": NH, "n_head_kv": NKV, "head_dim": D, "n_ctx": N_CTX, "n_past": n_past,
                   "types_qkvo": ["Q4_K", "Q4_K", "Q6_K", "Q4_K"]},
        "roofline": {"bound": "hbm", "achieved": round(abytes / dec_ev / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(abytes / dec_ev / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "qwmoe_attn_seg at T=1 (the segment's kernels together)",
                     "bytes_per_call": abytes, "weight_bytes": wbytes, "kv_bytes": kvbytes,
                     "avg_call_ms": round(dec_ev * 1e3, 4)},
        "prefill_chunk_512": {"n_past_0_ms": round(pre0_wall * 1e3, 4), "n_past_3584_ms": round(pre1_wall * 1e3, 4),
                              "tok_s_at_n_past_3584": round(512 / pre1_wall, 1)},
        "decode_hip_graph": {"ms_per_call": None if g_ms is None else round(g_ms, 4),
                             "tok_s": None if g_ms is None else round(1e3 / g_ms, 1),
                             "achieved_gbs": None if g_ms is None else round(abytes / g_ms / 1e6, 1),
                             "replay_equals_eager_bitwise": g_equal},
        "decoder_layer_decode": {"ms": round(lay_wall * 1e3, 4), "avg_call_ms": round(lay_ev * 1e3, 4),
                                 "bytes_per_call": abytes + moe_bytes,
                                 "achieved_gbs": round((abytes + moe_bytes) / lay_ev / 1e9, 1)},
        "cpu_baseline": cpu,
        "device_status": status,
    }
    print(json.dumps(line), flush=True)
    return 0


def gdn_bench(args) -> int:
    """The gated-delta-net half of Seg A (qwmoe_gdn_seg; build_gdn,
    core/runtime.cpp:737-859) at the shape of the reference's build_gdn comments:
    H = 2048, S = 128, 16 key and 16 value heads, d_conv = 4 (conv_ch 6144), Q4_K
    attn_qkv / ssm_out, Q6_K attn_gate, Q8_0 ssm_beta / ssm_alpha (seeded synthetic
    weights quantized on the GPU).  Timed: decode (T = 1, the states carried from
    call to call) -- the line's value, tokens per second of the segment -- and a
    prefill chunk of 512 tokens.  roofline: the weight rows one decode call reads
    plus the recurrent and conv states it reads and writes, over its time (HIP
    events).  cpu_baseline: ggml's own graph for the block (oracle/_ref, AVX-512
    build where the host has it) on the same weights at decode."""
    import numpy as np
    import torch
    from questwend_amd import Q4_K, Q6_K, Q8_0, ops, row_size

    S, HK, HV, DC = 128, 16, 16, 4
    d_inner, key_dim = HV * S, HK * S
    conv_ch = d_inner + 2 * key_dim
    types = (Q4_K, Q6_K, Q8_0, Q8_0, Q4_K)
    dev = "cuda:0"
    ops.init(0, 512 << 20)

    def qmat(rows, cols, t, seed):
        f = torch.empty((rows, cols), dtype=torch.float32, device=dev)
        ops.randn_(f, seed, 0.0, 0.02)
        return ops.quantize_chunk(t, f)

    def vec(n, seed, mean=1.0, std=0.1):
        v = torch.empty(n, dtype=torch.float32, device=dev)
        return ops.randn_(v, seed, mean, std)

    sd = args.seed * 1000 + 950
    w_qkv, w_gate = qmat(conv_ch, H, types[0], sd + 1), qmat(d_inner, H, types[1], sd + 2)
    w_beta, w_alpha = qmat(HV, H, types[2], sd + 3), qmat(HV, H, types[3], sd + 4)
    w_out = qmat(H, d_inner, types[4], sd + 5)
    an, fn, sn = vec(H, sd + 6), vec(H, sd + 7), vec(S, sd + 8)
    dtb = vec(HV, sd + 9, 0.0, 0.5)
    ssm_a = -(vec(HV, sd + 10, 1.25, 0.3).abs() + 0.1)
    conv1d = torch.empty((conv_ch, DC), dtype=torch.float32, device=dev)
    ops.randn_(conv1d, sd + 11, 0.0, 0.3)
    cs = torch.zeros((conv_ch, DC - 1), dtype=torch.float32, device=dev)
    ss = torch.zeros((HV, S, S), dtype=torch.float32, device=dev)
    GL = ops.make_gdn_layer(H, S, HK, HV, DC, types, an, w_qkv, w_gate, w_beta, w_alpha, w_out, dtb, ssm_a, conv1d,
                            sn, fn, cs, ss)
    torch.cuda.synchronize()

    def timed(fn_, n):
        for _ in range(max(2, args.warmup)):
            fn_()
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        t0 = time.perf_counter()
        for a, b in evs:
            a.record()
            fn_()
            b.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / n
        return wall, sum(a.elapsed_time(b) for a, b in evs) / n / 1000.0

    h1 = torch.empty((1, H), dtype=torch.float32, device=dev)
    ops.randn_(h1, sd + 20, 0.0, 1.0)
    hp = torch.empty((512, H), dtype=torch.float32, device=dev)
    ops.randn_(hp, sd + 21, 0.0, 1.0)
    dec_wall, dec_ev = timed(lambda: ops.gdn_seg(GL, h1), args.steps)
    pre_wall, pre_ev = timed(lambda: ops.gdn_seg(GL, hp), max(4, args.steps // 16))
    # the decode call captured into a HIP graph (the states advance on every
    # replay, as on every eager call); one replay checked against an eager call
    # from the same states
    g_ms, g_hold = graph_replay_ms(lambda: ops.gdn_seg(GL, h1), args.steps)
    g_equal = None
    if g_hold is not None:
        cs0, ss0 = cs.clone(), ss.clone()
        g_hold[0].replay()
        torch.cuda.synchronize()
        r_out, r_cs, r_ss = g_hold[1][0].clone(), cs.clone(), ss.clone()
        cs.copy_(cs0)
        ss.copy_(ss0)
        e_out = ops.gdn_seg(GL, h1)
        torch.cuda.synchronize()
        g_equal = bool(torch.equal(r_out, e_out[0]) and torch.equal(r_cs, cs) and torch.equal(r_ss, ss))
    status = ops.device_status(clear=True)

    wbytes = conv_ch * row_size(types[0], H) + d_inner * row_size(types[1], H) + HV * row_size(types[2], H) + \
        HV * row_size(types[3], H) + H * row_size(types[4], d_inner)
    sbytes = 2 * (HV * S * S + conv_ch * (DC - 1)) * 4
    abytes = wbytes + sbytes + (4 * H + S + conv_ch * DC + 2 * HV) * 4
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(ROOT / "tests"))
        from oracle_lib import REF_SO, REF_SO_AVX512, GdnWeights, RefGGML, have_ref_avx512
        if REF_SO.exists():
            gw = GdnWeights.__new__(GdnWeights)
            gw.H, gw.S, gw.H_k, gw.H_v, gw.d_conv, gw.types = H, S, HK, HV, DC, types
            gw.d_inner, gw.key_dim, gw.conv_ch = d_inner, key_dim, conv_ch
            gw.w_qkv, gw.w_gate, gw.w_beta, gw.w_alpha, gw.w_out = (t.cpu().numpy().reshape(-1) for t in
                                                                    (w_qkv, w_gate, w_beta, w_alpha, w_out))
            gw.attn_norm, gw.ffn_norm, gw.ssm_norm, gw.dt_bias, gw.ssm_a = (t.cpu().numpy() for t in
                                                                            (an, fn, sn, dtb, ssm_a))
            gw.conv1d = conv1d.cpu().numpy()
            csh, ssh = cs.cpu().numpy().copy(), ss.cpu().numpy().copy()
            x = h1.cpu().numpy()
            cpuinfo = host_cpu()
            n_thr = max(1, min(cpuinfo["cores_per_socket"], cpuinfo["cpus_available"]))
            ref = RefGGML(REF_SO_AVX512 if have_ref_avx512() else REF_SO)
            ref.gdn_seg(gw, x, csh, ssh, n_threads=n_thr)
            times, t_all = [], time.perf_counter()
            while (time.perf_counter() - t_all < 10.0 or len(times) < 5) and len(times) < 5000:
                t0 = time.perf_counter()
                ref.gdn_seg(gw, x, csh, ssh, n_threads=n_thr)
                times.append(time.perf_counter() - t0)
            med = float(np.median(times))
            cpu = {"value": round(1.0 / med, 1), "unit": "tok/s", "cores": n_thr, "kind": "reference",
                   "sample": f"{len(times)} decode steps (T=1, states carried) of ggml's gated-delta-net graph in "
                             f"{time.perf_counter() - t_all:.1f}s",
                   "median_ms_per_step": round(med * 1e3, 4), "isa": "AVX-512" if ref.isa() == 512 else "AVX2",
                   "threads": n_thr, "cpu": cpuinfo["model"]}
    line = {
        "metric": "gated-delta-net decode tok/s + achieved HBM GB/s, Seg A recurrent half (qwen3next / qwen35moe)",
        "value": round(1.0 / dec_wall, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dec_wall * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_K/q6_K/q8_0 x q8_K/q8_0 -> f32; f32 states",
        "data": "synthetic (seeded N(0,0.02) weights quantized on the GPU; N(0,1) inputs; states from zero)",
        "config": {"workload": "gated-delta-net half of Seg A (qwmoe_gdn_seg)", "n_embd": H, "d_state": S,
                   "n_group": HK, "dt_rank": HV, "d_conv": DC, "conv_ch": conv_ch,
                   "types_qkv_gate_beta_alpha_out": ["Q4_K", "Q6_K", "Q8_0", "Q8_0", "Q4_K"]},
        "roofline": {"bound": "hbm", "achieved": round(abytes / dec_ev / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(abytes / dec_ev / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "qwmoe_gdn_seg at T=1 (the segment's kernels together)",
                     "bytes_per_call": abytes, "weight_bytes": wbytes, "state_bytes": sbytes,
                     "avg_call_ms": round(dec_ev * 1e3, 4)},
        "prefill_chunk_512": {"ms": round(pre_wall * 1e3, 4), "avg_call_ms": round(pre_ev * 1e3, 4),
                              "tok_s": round(512 / pre_wall, 1)},
        "decode_hip_graph": {"ms_per_call": None if g_ms is None else round(g_ms, 4),
                             "tok_s": None if g_ms is None else round(1e3 / g_ms, 1),
                             "achieved_gbs": None if g_ms is None else round(abytes / g_ms / 1e6, 1),
                             "replay_equals_eager_bitwise": g_equal},
        "cpu_baseline": cpu,
        "device_status": status,
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--c5-layers", type=int, default=94,
                    help="config5: layers in the decode stack (configs[4] has 94; fewer only for counter runs)")
    ap.add_argument("--traffic", default=str(TRAFFIC_FILE),
                    help="text file whose 'hbm_bytes_per_launch = N' line is the HBM traffic of one decode "
                         "launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (copy-calibrated)")
    ap.add_argument("--copy-probe", action="store_true", help="run only the copy-kernel calibration probe")
    ap.add_argument("--workload", choices=["decode", "prefill", "expert_cache", "verify", "config5", "attn", "gdn"],
                    default="decode",
                    help="decode: configs[1] (the headline line); prefill: configs[2]; expert_cache: configs[1] "
                         "decode with the experts offloaded to pinned host memory; verify: configs[1] stack on "
                         "T = 1..--tokens verify batches; config5: configs[4] decode and prefill; attn: the "
                         "attention half of Seg A and a whole decoder layer at the 30B shape; gdn: the gated-delta-net half of Seg A")
    ap.add_argument("--resident", type=float, default=0.5, help="expert_cache: fraction of experts in HBM")
    ap.add_argument("--zipf", type=float, default=1.1, help="expert_cache: router skew (0: none)")
    ap.add_argument("--copy-engine", action="store_true",
                    help="expert_cache: every fetch by hipMemcpyAsync (no slab gather kernel)")
    ap.add_argument("--tokens", type=int, default=None, help="prefill batch size (512); verify: largest T (4)")
    ap.add_argument("--mfma-min-rows", type=int, default=1, help="prefill: experts with this many rows use MFMA")
    ap.add_argument("--exact-only", action="store_true",
                    help="prefill / config5: time only the default (exact) form, for kernel traces")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the sharding plan is "
              "documented, not built)", file=sys.stderr)
        return 2
    if args.tokens is None:
        args.tokens = 4 if args.workload == "verify" else 512
    if args.copy_probe:
        return copy_probe()
    if args.workload == "prefill":
        return prefill(args)
    if args.workload == "expert_cache":
        return expert_cache_bench(args)
    if args.workload == "verify":
        return verify_bench(args)
    if args.workload == "config5":
        return config5_bench(args)
    if args.workload == "gdn":
        return gdn_bench(args)
    if args.workload == "attn":
        return attn_bench(args)

    import numpy as np
    import torch
    from questwend_amd import Q4_K, ops, row_size

    ops.init(0, 256 << 20)
    t_gen = time.perf_counter()
    layers = make_weights(torch, ops, Q4_K, args.seed)
    t_gen = time.perf_counter() - t_gen
    Ls = [ops.make_layer(H, E, K_USED, F, r, g, u, d, (Q4_K,) * 3) for (r, g, u, d) in layers]
    stack = ops.DecodeStack(Ls, RMS_EPS, keepalive=layers)
    n_steps = args.steps + args.warmup
    xs = torch.empty((n_steps, H), dtype=torch.float32, device="cuda:0")
    ops.randn_(xs, args.seed + 777, 0.0, 1.0)
    out = torch.empty(H, dtype=torch.float32, device="cuda:0")
    xo = torch.empty(H, dtype=torch.float32, device="cuda:0")
    ids = torch.empty((N_LAYER, K_USED), dtype=torch.int32, device="cuda:0")
    wts = torch.empty((N_LAYER, K_USED), dtype=torch.float32, device="cuda:0")

    # untimed pass over the same tokens, keeping every step's output and ids
    # (the reference CPU backend is compared against these below)
    gpu_out = torch.empty((args.steps, H), dtype=torch.float32, device="cuda:0")
    gpu_ids = torch.empty((args.steps, N_LAYER, K_USED), dtype=torch.int32, device="cuda:0")
    for i in range(args.steps):
        stack.run(xs[args.warmup + i], gpu_out[i], xo, gpu_ids[i], wts)
    torch.cuda.synchronize()

    for i in range(args.warmup):
        stack.run(xs[i], out, xo)
    torch.cuda.synchronize()
    # per-launch HIP events on the launch stream (torch's current stream)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        evs[i][0].record()
        stack.run(xs[args.warmup + i], out, xo)
        evs[i][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = sum(a.elapsed_time(b) for a, b in evs) / args.steps
    status = stack.status()
    ms_per_step = wall * 1000.0 / args.steps
    tok_s = args.steps / wall
    abytes = algorithmic_bytes_per_token()
    achieved = abytes / (kern_ms / 1000.0) / 1e9
    traffic, traffic_note = measured_traffic(args.traffic)

    cpu, parity = None, None
    if not args.no_cpu_baseline:
        def gpu_layer(l, x):
            o, _, i2, _ = ops.ffn_layer(Ls[l], torch.from_numpy(x).to("cuda:0"), rms_eps=RMS_EPS)
            return o[0].cpu().numpy(), i2[0].cpu().numpy()

        cpu, parity = cpu_reference_stack(layers, xs.cpu().numpy(), args.warmup, gpu_out.cpu().numpy(),
                                          gpu_ids.cpu().numpy(), gpu_layer)

    line = {
        "metric": "decode tok/s + achieved HBM GB/s (% of 8 TB/s), Q4_K MoE FFN 30B-A3B",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_K x q8_K -> int32 -> f32",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q4_K on the GPU; N(0,1) token inputs)",
        "config": {"workload": "Qwen3-30B-A3B MoE FFN stack, 48 layers, batch-1 decode (configs[1])",
                   "n_embd": H, "n_expert": E, "n_expert_used": K_USED, "n_ff_exp": F, "n_layer": N_LAYER,
                   "weights": "Q4_K", "rms_eps": RMS_EPS,
                   "path": "qwmoe_decode_stack_run: one persistent launch per token, all 48 layers"},
        "hbm_gbs": round(abytes * tok_s / 1e9, 1),
        "hbm_frac": round(abytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": KERNEL_NAMES.get(stack.kernel(), "?") + " (one launch = one token through 48 layers)",
                     "bytes_per_launch": abytes, "avg_launch_ms": round(kern_ms, 4),
                     "traffic_source": traffic_note, "kernel_sources_sha256": kernel_sources_sha256()[:16]},
        "cpu_baseline": cpu,
        "parity_vs_reference_cpu": parity,
        "device_status": status,
        "weight_gen_s": round(t_gen, 2),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
