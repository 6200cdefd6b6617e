"""Benchmark of the MI355X G1 control step (BASELINE.json metric): ms per 20 ms control step and world-steps/s, forward
and forward+VJP, at 4096 worlds (and 16384), on one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--worlds 4096] [--no-cpu] [--no-16k] [--no-small]
                    [--no-configs] [--no-corpus] [--no-rounds]

A step is one control step (4 substeps of 5 ms, Newton 10 iterations) of B worlds of BASELINE config 1 (seeded
synthetic states, inputs resident in HBM before the timed region), exactly what torch_ffi.forward runs: the dispatch
order pre-pass and the forward kernel. The headline (`ms_per_step`, `value`): W untimed calls, then K calls back to
back between two synchronizations, timed with HIP events on the launch stream; rank 0 prints one JSON line.
Forward+VJP is the taped forward plus the adjoint (torch_ffi.forward(tape=True) + torch_ffi.backward), timed the same
way.

`rounds` restates the reference's timing protocol (scripts/paper_bench/common.py:1-10,154-187): a warm-up of at least
5 calls and 1 s, then 6 rounds of n back-to-back calls with one synchronization each (n chosen so that a round lasts
about 0.25 s, at most 200 calls), round 0 dropped; ms per call median / p10 / p90 / min / max over the 5 kept rounds.
It covers the forward and forward+VJP at 4096 and 16384 synthetic worlds (and at 512 and 1024: `worlds_512`,
`worlds_1024`, the other batch sizes the reference publishes, docs/results/paper_rtx6000/paper_bench.md:80-81, whose
numbers each of these entries carries) and at the 4096 states of the reference's corpus mf_s0 (`corpus_mf_s0`: the inputs its published 1.214 / 1.784 ms are measured on,
docs/results/paper_rtx6000/paper_bench.md:91-92; a committed fixture, tests/golden/corpus_mf_s0.npz).

Also reported: config 3 (`config3_jacobian`: full 71 x 99 step Jacobians of the 4096 worlds from one taped forward
and 71 VJPs, us per world-Jacobian) and config 4 (`config4_bptt`: a 32-step rollout of 16384 contact-heavy worlds with
backprop through time, checkpoint segments of 8 steps, and its capped world-steps).

`roofline` is the dominant kernel's, k_forward: algorithmic flops per launch (the float64 CPU restatement's
closed-form phase counts on the same inputs, counted once before timing, per world-step x B) divided by k_forward's
mean duration, timed live here with HIP events around K back-to-back launches of the forward alone
(dk_fwd_forward_ordered, cycling through 8 dispatch orders computed before: one order's kernel time differs from
another's by up to 2%, and the step computes a new order every call); peak is MI355X's FP32 (157.3 TFLOP/s). `traffic` is k_forward's HBM
bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE (the committed summary). `roofline_adjoint` is the same for
k_adjoint, the VJP's kernel: the float64 restatement's closed-form count of the adjoint's flops (default variant)
over k_adjoint's mean duration, timed live around back-to-back launches over 8 dispatch orders, and its HBM rate (the
tape read plus the adjoint's interface bytes) against 8 TB/s. `cpu_baseline` is the float64 CPU
restatement ("port"), timed with the same round protocol: one thread on the 64 worlds of config 0 (the reference's
single-thread CPU case) and, in `all_threads`, the host's usable cores (len(os.sched_getaffinity(0)), at most 16: the
GPU box's CPU share) on 4096 config-0 worlds (the reference's batched CPU case).
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# the reference's published ms per step (forward, fwd+VJP) on an RTX PRO 6000 Blackwell at each batch size,
# docs/results/paper_rtx6000/paper_bench.md:80-81
REF_RTX6000_MS = {512: {"forward": 0.609, "fwd_vjp": 0.797}, 1024: {"forward": 0.723, "fwd_vjp": 0.943},
                  4096: {"forward": 1.201, "fwd_vjp": 1.783}, 16384: {"forward": 3.962, "fwd_vjp": 5.938}}
METRIC = "ms per 20 ms control step @4096 worlds, forward and fwd+VJP; world-steps/s"
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
# interface bytes per world-step (inputs 556 B, outputs 440 B), the design-independent HBM traffic of the forward
IO_BYTES_FWD = (36 + 35 + 35 + 29 + 1 + 3) * 4 + (36 + 35 + 35) * 4 + 16
# HBM bytes per k_forward launch at 4096 worlds, measured with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (two runs,
# each scaled by the same counter's reading on a copy of known size, `--copy-mib`); the summary holds the command
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_forward_4096_traffic.md")
# the adjoint's interface bytes per world-step (cotangents 284 B and friction / com 16 B in, gradients 400 B and
# info 4 B out) and the tape it reads (4 substeps x 1472 float32 words)
IO_BYTES_VJP = (36 + 35 + 1 + 3) * 4 + (36 + 35 + 29) * 4 + 4
TAPE_BYTES = 4 * 1472 * 4
ORDERS = 8  # dispatch orders the kernel-alone timings cycle through
CORPUS = os.path.join(ROOT, "tests", "golden", "corpus_mf_s0.npz")
KEYS = ("qpos", "qvel", "warm", "ctrl", "friction", "com")
ROUNDS, WARM_CALLS, WARM_S, ROUND_S, MAX_CALLS = 5, 5, 1.0, 0.25, 200


def measured_traffic(worlds, key="traffic_bytes_per_launch"):
    """Bytes per launch from the committed traffic summary (line `<key>: N`; k_forward's by default,
    traffic_bytes_per_launch_adjoint for k_adjoint), or None when there is none for this world count."""
    if worlds != 4096 or not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith(key + ":"):
            return int(line.split(":")[1])
    return None


def _stats(per_call_ms, n, warm_calls, warm_s):
    a = np.asarray(per_call_ms)
    return {"median_ms": float(np.median(a)), "p10_ms": float(np.percentile(a, 10)),
            "p90_ms": float(np.percentile(a, 90)), "min_ms": float(a.min()), "max_ms": float(a.max()),
            "calls_per_round": n, "kept_rounds": len(a), "warmup_calls": warm_calls, "warmup_s": round(warm_s, 3)}


def protocol_cpu(call):
    """The reference's round protocol (common.py:154-187) for a host call: ms per call over the kept rounds."""
    t0, k = time.perf_counter(), 0
    while k < WARM_CALLS or time.perf_counter() - t0 < WARM_S:
        call()
        k += 1
    warm = time.perf_counter() - t0
    n = int(min(MAX_CALLS, max(1, round(ROUND_S * 6 / (warm / k)))))  # CPU rounds of about 1.5 s
    per = []
    for _ in range(ROUNDS + 1):
        t = time.perf_counter()
        for _ in range(n):
            call()
        per.append(1e3 * (time.perf_counter() - t) / n)
    return _stats(per[1:], n, k, warm)


def protocol_gpu(fn, stream):
    """The reference's round protocol for a GPU call: warm-up >= 5 calls and >= 1 s (synchronized), then 6 rounds of
    n back-to-back calls, each timed with HIP events on `stream` and one synchronization, round 0 dropped."""
    import torch
    t0, k = time.perf_counter(), 0
    while k < WARM_CALLS or time.perf_counter() - t0 < WARM_S:
        fn()
        torch.cuda.synchronize()
        k += 1
    warm = time.perf_counter() - t0
    n = int(min(MAX_CALLS, max(1, round(ROUND_S / (warm / k)))))
    per = []
    for _ in range(ROUNDS + 1):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / n)
    return _stats(per[1:], n, k, warm)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            return next(line.split(":", 1)[1].strip() for line in f if line.startswith("model name"))
    except (OSError, StopIteration):
        return "unknown CPU"


def cpu_baseline():
    """The float64 CPU restatement (test oracle) on config-0 states with the round protocol: one thread on 64 worlds,
    and the host's usable cores (at most 16) on 4096 worlds. world-steps/s from the median round."""
    import oracle
    from nablaengine_amd import synthetic
    st = synthetic.states(64, config=0, dtype=np.float64)
    one = protocol_cpu(lambda: oracle.step(**st, **oracle.ENGINE))
    threads = min(16, len(os.sched_getaffinity(0)))
    big = synthetic.states(4096, config=0, dtype=np.float64)
    many = protocol_cpu(lambda: oracle.step_mt(threads, **big, **oracle.ENGINE))
    settings = "float64 CPU restatement, not MuJoCo; Newton 10 it, tol 1e-8, line search 40 / 1e-7 (the engine's)"
    published = {"note": "the reference's MuJoCo C 3.17 timings on an AMD EPYC 9555, 16 threads allowed "
                         "(docs/results/paper_rtx6000/paper_bench.md:5,28-29), "
                         "not measured here: this port, with dense constraint Jacobians and 40 line-search "
                         "evaluations, is about 2.8x slower per thread than MuJoCo C, so a GPU / CPU ratio built on "
                         "it overstates the GPU's advantage by about as much",
                 "ms_64_worlds_1_thread": 8.591, "ms_4096_worlds_16_threads": 34.746}
    return dict(value=64e3 / one["median_ms"], unit="world-steps/s", cores=1, kind="port", cpu=_cpu_model(),
                host_threads=len(os.sched_getaffinity(0)), published_mujoco=published,
                sample=f"64 config-0 worlds per call, {one['calls_per_round']} calls per round, 5 kept rounds "
                       f"({settings}); ms per 64-world step median {one['median_ms']:.2f}",
                rounds=one,
                all_threads=dict(value=4096e3 / many["median_ms"], unit="world-steps/s", cores=threads,
                                 sample=f"4096 config-0 worlds per call on {threads} threads (contiguous shares), "
                                        f"{many['calls_per_round']} calls per round, 5 kept rounds; ms per "
                                        f"4096-world step median {many['median_ms']:.1f}",
                                 rounds=many))


def algorithmic_flops(st):
    """Mean algorithmic flops per world-step of these states (closed-form counts of the float64 restatement)."""
    import oracle
    r = oracle.step(**{k: v.astype(np.float64) for k, v in st.items()}, **oracle.ENGINE, flops=True)
    return float(np.mean(r[4]))


def algorithmic_flops_vjp(st):
    """Mean algorithmic flops per world-step of the VJP of these states' steps (the interface's default variant,
    clamp_kv 0, normal 3; closed-form counts of the float64 restatement's adjoint)."""
    import oracle
    from nablaengine_amd import synthetic, torch_ffi
    s64 = {k: v.astype(np.float64) for k, v in st.items()}
    cq, cv = (x.astype(np.float64) for x in synthetic.cotangents(len(st["qpos"])))
    r = oracle.vjp(**s64, g_qpos=cq, g_qvel=cv, clamp_kv=torch_ffi.CLAMP_KV, normal=torch_ffi.NORMAL,
                   **oracle.ENGINE, flops=True)
    return float(np.mean(r[3]))


def timed(fn, steps, warmup, stream):
    """Mean ms per call of fn over `steps` back-to-back calls (HIP events on `stream`), after `warmup` calls."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _calls(st):
    """(forward call, forward+VJP call, the output holder) on states st, inputs resident on the GPU."""
    import torch
    from nablaengine_amd import synthetic, torch_ffi
    B = len(st["qpos"])
    args = [torch.from_numpy(np.ascontiguousarray(st[k], np.float32)).cuda() for k in KEYS]
    gq, gv = (torch.from_numpy(x).cuda() for x in synthetic.cotangents(B))
    out = {}

    def fwd():
        out["r"] = torch_ffi.forward(*args)

    def vjp():
        r = torch_ffi.forward(*args, tape=True)
        torch_ffi.backward(r[4], args[4], args[5], gq, gv)
    return fwd, vjp, out, args


def measure(B, steps, warmup, kernel=False, rounds=True):
    """(forward ms, fwd+VJP ms, k_forward ms or None, k_adjoint ms or None, info of the last forward, round-protocol
    stats or None) at B worlds of config 1."""
    import torch
    from nablaengine_amd import synthetic, torch_ffi
    st = synthetic.states(B, config=1)
    fwd, vjp, out, args = _calls(st)
    stream = torch.cuda.current_stream()
    ms = timed(fwd, steps, warmup, stream)
    info = out["r"][3].cpu().numpy()
    vjp_ms = timed(vjp, steps, warmup, stream)
    kms = ams = None
    if kernel:
        # k_forward alone: ORDERS dispatch orders computed first, then ordered launches back to back, cycling through
        # them. An order's ties within a cost bucket fall as its atomics do, and one order's kernel time differs from
        # another's by up to 2% (the XCDs' queues get different worlds); the step computes a new order every call,
        # so the kernel's time is taken over several, as the step sees it
        lib = torch_ffi.load_library()
        st_ = ctypes.c_void_p(stream.cuda_stream)
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        kw = dict(dtype=torch.float32, device="cuda")
        q1, v1, w1 = torch.empty((B, 36), **kw), torch.empty((B, 35), **kw), torch.empty((B, 35), **kw)
        inf = torch.empty((B, 4), dtype=torch.int32, device="cuda")
        works = [torch.empty((int(lib.dk_fwd_work_bytes(B)),), dtype=torch.uint8, device="cuda")
                 for _ in range(ORDERS)]
        for work in works:
            assert lib.dk_fwd_order(st_, B, p(args[0]), p(work)) == 0
        nk = [0]

        def kern():
            work = works[nk[0] % ORDERS]
            nk[0] += 1
            assert lib.dk_fwd_forward_ordered(st_, B, *map(p, args), 10, 4, p(q1), p(v1), p(w1), p(inf), None, None,
                                              p(work)) == 0
        kms = timed(kern, max(steps, 2 * ORDERS), warmup, stream)
        # k_adjoint alone: one tape and ORDERS adjoint orders, then the ordered launches back to back, cycling
        # through them, with the diagnostic counting on (as torch_ffi.backward launches it)
        tape = torch_ffi.forward(*args, tape=True)[4]
        gq, gv = (torch.from_numpy(x).cuda() for x in synthetic.cotangents(B))
        bq, bv, bu = torch.empty((B, 36), **kw), torch.empty((B, 35), **kw), torch.empty((B, 29), **kw)
        binf = torch.empty((B,), dtype=torch.int32, device="cuda")
        aworks = [torch.empty((int(lib.dk_adjoint_work_bytes(B)),), dtype=torch.uint8, device="cuda")
                  for _ in range(ORDERS)]
        counters = torch.zeros(len(torch_ffi.DIAG), dtype=torch.int64, device="cuda")
        for awork in aworks:
            assert lib.dk_adjoint_order(st_, B, 4, p(tape), p(awork)) == 0
        na = [0]

        def adj():
            awork = aworks[na[0] % ORDERS]
            na[0] += 1
            assert lib.dk_adjoint_work_ordered(st_, B, 4, p(tape), p(args[4]), p(args[5]), p(gq), p(gv), p(bq), p(bv),
                                               p(bu), p(binf), None, 0.0, torch_ffi.CLAMP_KV, torch_ffi.NORMAL,
                                               p(awork), p(counters)) == 0
        ams = timed(adj, max(steps, 2 * ORDERS), warmup, stream)
    rs = {"forward": protocol_gpu(fwd, stream), "fwd_vjp": protocol_gpu(vjp, stream)} if rounds else None
    return ms, vjp_ms, kms, ams, info, rs


def measure_corpus():
    """The forward and forward+VJP of the reference corpus mf_s0's 4096 states (warm start as stored), with the
    round protocol."""
    import torch
    z = np.load(CORPUS)
    st = {k: z["qacc_warmstart" if k == "warm" else k] for k in KEYS}
    fwd, vjp, out, _ = _calls(st)
    stream = torch.cuda.current_stream()
    rf, rv = protocol_gpu(fwd, stream), protocol_gpu(vjp, stream)
    info = out["r"][3].cpu().numpy()
    return {"worlds": len(st["qpos"]), "inputs": "benchmarks/data/mf_s0.npz (4096 corpus states: qpos, qvel, "
                                                  "qacc_warmstart, ctrl, friction, com; cotangents N(0, 1))",
            "ms_per_step": rf["median_ms"], "ms_per_step_fwd_vjp": rv["median_ms"],
            "world_steps_per_s": 4096e3 / rf["median_ms"], "world_steps_per_s_fwd_vjp": 4096e3 / rv["median_ms"],
            "reference_rtx_pro_6000_ms": {"forward": 1.214, "fwd_vjp": 1.784},
            "forward": rf, "fwd_vjp": rv,
            "capacity": {"contacts_max": int(info[:, 1].max()), "rows_max": int(info[:, 2].max()),
                         "overflow_worlds": int(((info[:, 3] & 20) != 0).sum())}}


def measure_jacobian(B, reps=2):
    """ms per batch of B full step Jacobians (one taped forward + 71 VJPs on its tape) and us per
    world-Jacobian."""
    import torch
    from nablaengine_amd import rollout, synthetic
    st = synthetic.states(B, config=1)
    args = [torch.from_numpy(st[k]).cuda() for k in KEYS]
    ms = timed(lambda: rollout.jacobian(*args), reps, 1, torch.cuda.current_stream())
    return {"worlds": B, "ms_per_batch": ms, "us_per_world_jacobian": 1e3 * ms / B,
            "method": "1 taped forward + 71 one-hot VJPs on that tape (the reference's), rows qpos' (36) and qvel' "
                      "(35), columns qpos tangent (35), qvel (35), ctrl (29)"}


def measure_bptt(B, T=32, k=8):
    """a T-step rollout of B contact-heavy worlds with backprop through time, segments of k steps
    recomputed in the backward; ms per rollout (forward + backward) and the capped world-steps of its forward."""
    import torch
    from nablaengine_amd import rollout, synthetic, torch_ffi
    st = synthetic.states(B, config=4)
    us = torch.from_numpy(synthetic.ctrl_sequence(T, B)).cuda()
    g = {k_: torch.from_numpy(st[k_]).cuda() for k_ in KEYS}

    def run():
        q = g["qpos"].clone().requires_grad_(True)
        v = g["qvel"].clone().requires_grad_(True)
        u = us.clone().requires_grad_(True)
        states = rollout.rollout(q, v, g["warm"], u, g["friction"], g["com"], checkpoint_every=k)
        loss = sum((qt[:, 2] ** 2).sum() + 0.01 * (vt ** 2).sum() for qt, vt in states)
        loss.backward()
    ms = timed(run, 1, 1, torch.cuda.current_stream())
    # the capped world-steps of the rollout's forward (info[:, 3] & (4 | 16)), from a forward-only pass
    q, v, w = g["qpos"], g["qvel"], g["warm"]
    capped = contacts_max = rows_max = 0
    for t in range(T):
        q, v, w, info = torch_ffi.forward(q, v, w, us[t], g["friction"], g["com"])
        i = info.cpu().numpy()
        capped += int(((i[:, 3] & 20) != 0).sum())
        contacts_max, rows_max = max(contacts_max, int(i[:, 1].max())), max(rows_max, int(i[:, 2].max()))
    return {"worlds": B, "steps": T, "checkpoint_every": k, "ms_per_rollout_fwd_bwd": ms,
            "world_steps_per_s_fwd_bwd": B * T * 1e3 / ms, "capped_world_steps": capped,
            "contacts_max": contacts_max, "rows_max": rows_max}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--worlds", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-16k", action="store_true", help="skip the 16384-world forward and fwd+VJP lines")
    ap.add_argument("--no-small", action="store_true", help="skip the 512- and 1024-world forward and fwd+VJP lines")
    ap.add_argument("--no-configs", action="store_true", help="skip the config 3 (Jacobian) and 4 (BPTT) lines")
    ap.add_argument("--no-corpus", action="store_true", help="skip the mf_s0 corpus line")
    ap.add_argument("--no-rounds", action="store_true", help="skip the round-protocol statistics")
    ap.add_argument("--flop-sample", type=int, default=512, help="worlds the flop count is taken on")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="before the timed steps, copy a buffer of this many MiB 3 times (a kernel of known HBM "
                         "traffic that calibrates rocprofv3's FETCH_SIZE and WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: --gpus {a.gpus}: this build measures one GPU only (the worlds are independent; a multi-GPU "
              "run is B/G worlds per GPU with no exchange inside a step)", file=sys.stderr)
        sys.exit(2)
    import torch
    from nablaengine_amd import synthetic, torch_ffi
    torch_ffi.init(0)
    if a.copy_mib:
        src = torch.ones(a.copy_mib << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    B = a.worlds
    ms, vjp_ms, kms, ams, info, rs = measure(B, a.steps, a.warmup, kernel=True, rounds=not a.no_rounds)
    big = None
    if not a.no_16k and B != 16384:
        bms, bvjp, _, _, binfo, brs = measure(16384, max(a.steps // 4, 3), max(a.warmup // 4, 2),
                                              rounds=not a.no_rounds)
        big = {"worlds": 16384, "ms_per_step": bms, "ms_per_step_fwd_vjp": bvjp,
               "world_steps_per_s": 16384e3 / bms, "world_steps_per_s_fwd_vjp": 16384e3 / bvjp,
               "reference_rtx_pro_6000_ms": REF_RTX6000_MS[16384]}
        if brs:
            big["rounds"] = brs
    small = {}
    if not a.no_small:
        for b in (512, 1024):
            if b == B:
                continue
            sms, svjp, _, _, _, srs = measure(b, a.steps, a.warmup, rounds=not a.no_rounds)
            small[b] = {"worlds": b, "ms_per_step": sms, "ms_per_step_fwd_vjp": svjp,
                        "world_steps_per_s": b * 1e3 / sms, "world_steps_per_s_fwd_vjp": b * 1e3 / svjp,
                        "reference_rtx_pro_6000_ms": REF_RTX6000_MS[b]}
            if srs:
                small[b]["rounds"] = srs
    st = synthetic.states(B, config=1)
    sub = {k: v[: a.flop_sample] for k, v in st.items()}
    fl = algorithmic_flops(sub)
    achieved = fl * B / (kms * 1e-3) / 1e12
    fla = algorithmic_flops_vjp(sub)
    adj_achieved = fla * B / (ams * 1e-3) / 1e12
    adj_bytes = TAPE_BYTES + IO_BYTES_VJP  # per world-step: the tape read plus the adjoint's interface bytes
    res = {
        "metric": METRIC, "value": B * 1e3 / ms, "unit": "world-steps/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (BASELINE config 1: seeded standing states, random ctrl; model g1_train.mjb)",
        "config": {"workload": f"G1 control step forward, {B} worlds, 4 x 5 ms substeps, Newton 10 it, implicitfast",
                   "worlds": B, "substeps": 4, "iterations": 10},
        "ms_per_step_fwd_vjp": vjp_ms,
        "world_steps_per_s_fwd_vjp": B * 1e3 / vjp_ms,
        "ms_k_forward": kms,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_FP32_TFLOPS, "traffic": measured_traffic(B),
                     "note": "FP32 vector (VALU) work, no MFMA in the Newton path's bulk: achieved = closed-form "
                             f"algorithmic flops ({fl:.3g} per world-step, float64 restatement on {len(sub['qpos'])} "
                             "of the worlds) x worlds / k_forward's mean duration (HIP events around back-to-back "
                             "launches of the forward kernel alone over 8 dispatch orders, its stream); the step also "
                             "runs the dispatch-order pre-pass (ms_per_step - ms_k_forward)"},
        "roofline_hbm": {"achieved": IO_BYTES_FWD * B / (kms * 1e-3) / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": IO_BYTES_FWD * B / (kms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                         "note": f"interface bytes {IO_BYTES_FWD} per world-step"},
        "ms_k_adjoint": ams,
        "roofline_adjoint": {"bound": "mfma", "achieved": adj_achieved, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                             "frac": adj_achieved / PEAK_FP32_TFLOPS,
                             "traffic": measured_traffic(B, "traffic_bytes_per_launch_adjoint"),
                             "hbm": {"achieved": adj_bytes * B / (ams * 1e-3) / 1e9, "peak": PEAK_HBM_GBS,
                                     "unit": "GB/s", "frac": adj_bytes * B / (ams * 1e-3) / 1e9 / PEAK_HBM_GBS,
                                     "bytes_per_world_step": adj_bytes},
                             "note": "k_adjoint, the VJP's kernel (FP32 vector work, no MFMA): achieved = closed-form "
                                     "algorithmic flops of the VJP (" f"{fla:.3g}"
                                     " per world-step, the float64 restatement's adjoint count on "
                                     f"{len(sub['qpos'])} of the worlds, default variant) x worlds / k_adjoint's mean "
                                     "duration (HIP events around back-to-back launches over 8 dispatch orders, its "
                                     "stream); hbm: the tape read (4 substeps x 1472 words) plus the interface's "
                                     f"{IO_BYTES_VJP} bytes per world-step over the same duration"},
        "capacity": {"contacts_max": int(info[:, 1].max()), "rows_max": int(info[:, 2].max()),
                     "overflow_worlds": int(((info[:, 3] & 20) != 0).sum())},
    }
    if rs:
        res["rounds"] = dict(rs, protocol="scripts/paper_bench/common.py:154-187: warm-up >= 5 calls and >= 1 s, "
                                          "6 rounds of n calls (one synchronization each), round 0 dropped")
    if big:
        res["worlds_16384"] = big
    for b, v in small.items():
        res[f"worlds_{b}"] = v
    if not a.no_corpus and os.path.exists(CORPUS):
        res["corpus_mf_s0"] = measure_corpus()
    if not a.no_configs:
        res["config3_jacobian"] = measure_jacobian(B)
        res["config4_bptt"] = measure_bptt(16384)
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res))


if __name__ == "__main__":
    main()
