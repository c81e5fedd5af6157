#!/usr/bin/env python3
"""Benchmark of the MI355X S6 selective scan; prints ONE JSON line on stdout.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload fwd1|fwdbwd3|fwd2|fwdbwd4|mixer1|mamba3|decode|ssd2|copyref]

Default workload ``fwd1``: the forward scan at B=32, L=4096, D=256, N=16, bf16 I/O with
fp32 state (the configuration the headline metric is quoted on), called like a [B, L, D]
producer would: ``selective_scan_fn(x.mT, delta.mT, A, B.mT, C.mT, D=D,
return_last_state=True)``.  ``fwdbwd3`` times forward + backward at B=8, L=8192, D=768,
N=16 bf16; ``fwd2`` the fp32 N=64 long-sequence forward; ``fwdbwd4`` the packed varlen
forward + backward; ``mixer1`` the SSMMixer S6 core at the fwd1 shape; ``mamba3`` one
training step of the fused Mamba block (MambaInnerFn) at the fwdbwd3 shape; ``decode`` the
selective_state_update decode step (batch 64, d_inner 1536), graph-launched; ``ssd2`` the
Mamba-2 SSD (mamba_chunk_scan_combined) forward and forward + backward at Mamba-2 defaults.

* value: algorithmic HBM bytes of one step (each tensor once) / wall time per step, with
  the inputs resident in HBM.  Three independent input sets rotate so the 256 MB
  Infinity Cache cannot hold the working set.
* roofline: the dominant kernel (the fused scan/output kernel) timed live with HIP events
  that the library records on its own stream around that kernel.
* cpu_baseline: the CPU restatement of the reference path (selective_scan_ref, op for op,
  oracle/selective_scan_ref.py) timed on the host cores on a bounded sample of the same
  workload.
* fwd_bwd (fwd1 only, unless --no-fwdbwd): the config-3 training-shape forward + backward
  measured the same way, since the metric covers both; ``value`` stays the forward's.
Only one GPU is used: --gpus above 1 exits with a message.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ml-experiments_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "scan fwd / fwd+bwd achieved HBM GB/s (% of peak) and Mtok·ch/s at 1 GPU"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="fwd1",
                    choices=["fwd1", "fwdbwd3", "fwd2", "fwdbwd4", "mixer1", "mamba3",
                             "decode", "ssd2", "copyref"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fwdbwd", action="store_true",
                    help="fwd1 only: skip the config-3 fwd+bwd measurement carried in its line")
    ap.add_argument("--layout", default="channel_last", choices=["channel_last", "l_contiguous"],
                    help="scan workloads: [B, D, L] arguments as channel-last views of [B, L, D] "
                         "tensors (default), or L-contiguous tensors as the reference's zoology "
                         "Mamba passes them")
    return ap.parse_args()


def cpu_model():
    """The host CPU's model name, reported next to the CPU baseline so that its figure can be
    read against the hardware it ran on."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_config0_one_thread(make_inputs):
    """Config 0 (the reference's own CPU-runnable case: B=1, L=1024, D=128, N=16, fp32
    forward) through the restated reference path on 1 thread, median of 3."""
    import torch
    from s6scan.configs import CONFIGS
    from oracle.selective_scan_ref import selective_scan_ref
    cfg = CONFIGS[0]
    inp = make_inputs(cfg)
    args = (inp["x"].mT, inp["delta"].mT, inp["A"], inp["B"].mT, inp["C"].mT)
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        selective_scan_ref(*args, D=inp["D"], return_last_state=True)
        ts = []
        for _ in range(3):
            t = time.perf_counter()
            selective_scan_ref(*args, D=inp["D"], return_last_state=True)
            ts.append(time.perf_counter() - t)
    finally:
        torch.set_num_threads(prev)
    sec = statistics.median(ts)
    return {"seconds": round(sec, 4), "GB_per_s": round(cfg.algorithmic_bytes() / sec / 1e9, 5),
            "threads": 1}


def cpu_baseline(cfg, make_inputs, mixer=False, one_thread=True, target_s=3.0):
    """Reference CPU path on a bounded sample of the workload, about 10-20 s of host work.
    Forward workloads: whole sequences at the workload's seqlen, one call per sequence; a
    warm-up call on one sequence sets how many (up to the workload's batch) make one timed
    run last about ``target_s``; the median of 3 timed runs is reported.  Fwd+bwd workloads:
    one sequence of 1024 steps per call, since the restated path's backward (autograd through
    the per-step loop, ops/selective_scan_interface.py:138-139, where each step's index of deltaA
    materialises a full-size gradient) costs O(L^2) per sequence and a full-length sequence
    would take hours.  The scan workloads time the torch restatement of selective_scan_ref
    (op for op); the mixer workload the restatement of the reference SSMMixer's own scan loop
    (backbone.py:1207-1242, state in the input dtype as there)."""
    import dataclasses

    import torch
    from oracle.selective_scan_ref import selective_scan_ref, selective_scan_ref_grads
    from oracle.ssm_mixer_ref import ssm_mixer_scan_ref
    torch.set_num_threads(os.cpu_count() or 1)
    seqlen = 1024 if cfg.backward else (cfg.seqlen or 8192)
    nmax = cfg.batch if cfg.seqlen else 64
    one = dataclasses.replace(cfg, batch=1, seqlen=seqlen, nseq=0)

    def seq_inputs(i):
        inp = make_inputs(dataclasses.replace(one, seed=cfg.seed + i))
        mix = (mixer_extras(torch, inp, torch.Generator("cpu").manual_seed(7 + i))
               if mixer else None)
        return inp, mix

    def call(inp, mix):
        args = (inp["x"].mT, inp["delta"].mT, inp["A"], inp["B"].mT, inp["C"].mT)
        if mixer:
            ssm_mixer_scan_ref(inp["x"], mix["dt_raw"], mix["A_log"], mix["B"], mix["C"],
                               inp["D"], mix["z"])
        elif cfg.backward:
            selective_scan_ref_grads(*args, inp["D"], inp["dy"].mT)
        else:
            selective_scan_ref(*args, D=inp["D"], return_last_state=True)

    first = seq_inputs(0)
    t = time.perf_counter()
    call(*first)  # warm-up, also sizes the sample
    t1 = time.perf_counter() - t
    n = max(1, min(nmax, round(target_s / max(t1, 1e-6))))
    seqs = [first] + [seq_inputs(i) for i in range(1, n)]
    ts = []
    for _ in range(3):
        t = time.perf_counter()
        for inp, mix in seqs:
            call(inp, mix)
        ts.append(time.perf_counter() - t)
    sec = statistics.median(ts)
    sample_bytes = n * one.algorithmic_bytes()
    if mixer:  # + z read, + the gated output, as in the GPU line
        sample_bytes += 2 * n * seqlen * cfg.dim * first[0]["x"].element_size()
    return {
        "value": round(sample_bytes / sec / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"restated reference CPU path ("
                   f"{'SSMMixer scan loop' if mixer else 'selective_scan_ref'} op for op"
                   f"{' + autograd backward' if cfg.backward else ''}) on {n} sequence(s) of "
                   f"{cfg.name}, one call each: seqlen {seqlen}, dim {cfg.dim}, dstate "
                   f"{cfg.dstate}; median of 3 runs = {sec:.3f} s (warm-up call on one "
                   f"sequence {t1:.3f} s); os.cpu_count() = {os.cpu_count()}"),
        "mtok_ch_per_s": round(n * seqlen * cfg.dim / sec / 1e6, 4),
        "cpu_model": cpu_model(),
        **({"config0_one_thread": cpu_config0_one_thread(make_inputs)} if one_thread else {}),
    }


def mixer_extras(torch, inp, g):
    """Inputs of the SSMMixer-shaped workload, derived from a scan workload's inputs the
    way the reference mixer produces them (backbone.py:1185-1209): z is the second half of
    the in_proj output, B and C are slices of the x_proj output [B, L, dt_rank + 2N], dt is
    the dt_proj output before softplus, A = -exp(A_log)."""
    Bsz, L, D = inp["x"].shape
    N = inp["A"].shape[1]
    R = 16
    dev, dt = inp["x"].device, inp["x"].dtype
    xz = torch.randn(Bsz, L, 2 * D, generator=g).to(dt).to(dev)
    params = torch.empty(Bsz, L, R + 2 * N, dtype=dt, device=dev)
    params[..., R:R + N] = inp["B"]
    params[..., R + N:] = inp["C"]
    dt_raw = (0.5 * torch.randn(Bsz, L, D, generator=g) - 1.0).to(dt).to(dev)
    return {"z": xz.chunk(2, dim=-1)[1], "B": params[..., R:R + N], "C": params[..., R + N:],
            "dt_raw": dt_raw, "A_log": torch.log(-inp["A"])}


MAMBA3 = dict(batch=8, seqlen=8192, d_model=384, d_state=16, d_conv=4)


def mamba_block(torch, batch, seqlen, d_model, d_state, d_conv, dev, seed=0):
    """Random-init parameters of a zoology Mamba layer (mamba.py:22-100: expand 2,
    dt_rank = ceil(d_model / 16), S4D-real A, dt bias from U[1e-3, 1e-1])."""
    d_inner = 2 * d_model
    R = -(-d_model // 16)
    g = torch.Generator("cpu").manual_seed(seed)
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(dev).requires_grad_(True)
    dt = torch.exp(torch.rand(d_inner, generator=g) * (torch.log(torch.tensor(0.1))
                                                      - torch.log(torch.tensor(1e-3)))
                   + torch.log(torch.tensor(1e-3)))
    return dict(
        in_proj_weight=r(2 * d_inner, d_model, sc=d_model ** -0.5),
        conv1d_weight=r(d_inner, 1, d_conv, sc=d_conv ** -0.5), conv1d_bias=r(d_inner, sc=0.1),
        x_proj_weight=r(R + 2 * d_state, d_inner, sc=d_inner ** -0.5),
        delta_proj_weight=r(d_inner, R, sc=R ** -0.5),
        out_proj_weight=r(d_model, d_inner, sc=d_inner ** -0.5),
        A_log=torch.log(torch.arange(1, d_state + 1, dtype=torch.float32)).repeat(d_inner, 1)
        .to(dev).requires_grad_(True),
        D=torch.ones(d_inner, device=dev, requires_grad=True),
        delta_bias=(dt + torch.log(-torch.expm1(-dt))).to(dev).requires_grad_(True))


def mamba_cpu_baseline(torch, cfg):
    """The restated reference block (mamba_inner_ref, oracle/mamba_inner_ref.py) forward +
    autograd backward in fp32 on the host cores, batch 1, seqlen 256 (the restated scan is
    a Python loop over steps, about 8 s per run here)."""
    from oracle.mamba_inner_ref import mamba_inner_ref
    torch.set_num_threads(os.cpu_count() or 1)
    L = 256
    p = mamba_block(torch, 1, L, cfg["d_model"], cfg["d_state"], cfg["d_conv"], "cpu")
    h = torch.randn(1, L, cfg["d_model"])

    def run():
        xz = (p["in_proj_weight"] @ h[0].t()).unsqueeze(0)
        out = mamba_inner_ref(xz, p["conv1d_weight"], p["conv1d_bias"], p["x_proj_weight"],
                              p["delta_proj_weight"], p["out_proj_weight"], None,
                              -torch.exp(p["A_log"]), None, None, p["D"],
                              delta_bias=p["delta_bias"], delta_softplus=True)
        out.sum().backward()

    ts = []
    for _ in range(3):
        t = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t)
    sec = statistics.median(ts)
    d_inner = 2 * cfg["d_model"]
    return {"value": round(L * d_inner / sec / 1e6, 4), "unit": "Mtok·ch/s",
            "cores": torch.get_num_threads(), "kind": "port", "cpu_model": cpu_model(),
            "sample": (f"restated reference block (mamba_inner_ref: nn.Conv1d path, "
                       f"selective_scan_ref op for op, autograd backward), fp32, batch 1, "
                       f"seqlen {L}, d_model {cfg['d_model']}; median of 3 runs = {sec:.3f} s")}


def run_mamba(torch, args):
    """Workload mamba3: one training step (forward + backward) of the fused Mamba block
    (s6scan.mamba_inner.mamba_inner_fn, the reference's MambaInnerFn path, mamba.py:138-153)
    under bf16 autocast: in_proj, HIP causal conv1d + SiLU, x_proj / dt_proj GEMMs, HIP
    selective scan (softplus, D, z gate), out_proj, and the backward of all of it."""
    from s6scan import mamba_inner
    c = MAMBA3
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, L, dm, N = c["batch"], c["seqlen"], c["d_model"], c["d_state"]
    d_inner = 2 * dm
    sets = []
    for s in range(2):  # two rotating input sets
        g = torch.Generator("cpu").manual_seed(100 + s)
        sets.append((torch.randn(B, L, dm, generator=g).to(dev, torch.bfloat16),
                     torch.randn(B, L, dm, generator=g).to(dev, torch.bfloat16)))
    p = mamba_block(torch, B, L, dm, N, c["d_conv"], dev)

    def step(i):
        h, dy = sets[i % len(sets)]
        with torch.autocast("cuda", dtype=torch.bfloat16):
            # in_proj as mamba_inner.mamba_forward issues it (weight gradient split over tokens)
            xz = mamba_inner.InProjFn.apply(h.reshape(B * L, dm), p["in_proj_weight"],
                                            None).view(B, L, -1).mT
            out = mamba_inner.mamba_inner_fn(
                xz, p["conv1d_weight"], p["conv1d_bias"], p["x_proj_weight"],
                p["delta_proj_weight"], p["out_proj_weight"], None, -torch.exp(p["A_log"]),
                None, None, p["D"], delta_bias=p["delta_bias"], delta_softplus=True)
        out.backward(dy)
        for t in p.values():
            t.grad = None

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    K = args.steps
    mk = lambda: torch.cuda.Event(enable_timing=True)
    evs = [(mk(), mk()) for _ in range(K)]
    stream = torch.cuda.current_stream()
    for pair in evs:
        for e in pair:
            e.record(stream)
    g0, g1 = mk(), mk()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g0.record(stream)
    for i in range(K):
        mamba_inner.KERNEL_EVENTS = evs[i]
        step(i)
    g1.record(stream)
    torch.cuda.synchronize()
    mamba_inner.KERNEL_EVENTS = None
    ms_step = (time.perf_counter() - t0) * 1e3 / K
    kb_ms = statistics.mean(a.elapsed_time(b) for a, b in evs)
    # bwd_scan algorithmic bytes (each tensor once): u, delta, dout, z, out read and du,
    # ddelta, dz, out_z written (bf16); B, C read (bf16) and dB, dC written (fp32); A, D,
    # delta_bias in and their gradients out (fp32).
    E = B * L * d_inner
    kb_bytes = E * 2 * 9 + B * L * N * (2 + 2 + 4 + 4) + 2 * (4 * d_inner * N + 8 * d_inner)
    achieved = kb_bytes / (kb_ms * 1e-3) / 1e9
    res = {
        "metric": "fused Mamba block (MambaInnerFn) fwd+bwd Mtok·ch/s at 1 GPU",
        "value": round(B * L * d_inner / (ms_step * 1e-3) / 1e6, 2),
        "unit": "Mtok·ch/s", "n_gpus": 1, "steps": K, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded normal hidden states and output gradients; random-init "
                "parameters of a zoology Mamba layer)",
        "config": {"workload": (f"mamba3: zoology Mamba fast path, batch {B}, seqlen {L}, "
                                f"d_model {dm}, d_inner {d_inner}, d_state {N}, d_conv "
                                f"{c['d_conv']}, bf16 autocast, fwd+bwd")},
        "gpu_event_ms_per_step": round(g0.elapsed_time(g1) / K, 5),
        "roofline": {"kernel": "bwd_scan (softplus, z gate, out_z recompute)", "bound": "hbm",
                     "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": None,
                     "kernel_ms": round(kb_ms, 5)},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        res["cpu_baseline"] = mamba_cpu_baseline(torch, c)
    print(json.dumps(res), flush=True)


DECODE = dict(batch=64, dim=1536, dstate=16, steps_per_graph=16)


def run_decode(torch, args):
    """Workload decode: the recurrent decode step (s6scan.selective_state_update, the
    reference's selective_state_update, selective_state_update.py:121-201) of a Mamba layer
    with d_inner 1536 for 64 sequences: fp32 state updated in place, bf16 x / dt / z / B / C,
    softplus(dt + dt_bias), D and the z gate.  16 consecutive steps (each with its own inputs)
    are captured in one HIP graph, as a serving loop runs them, and the graph is replayed."""
    from s6scan.selective_state_update import selective_state_update
    c = DECODE
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, D, N, S = c["batch"], c["dim"], c["dstate"], c["steps_per_graph"]
    g = torch.Generator("cpu").manual_seed(5)
    r = lambda *sh, dt=torch.float32: torch.randn(*sh, generator=g).to(dev, dt)
    bf = torch.bfloat16
    state = r(B, D, N)
    A = -torch.exp(r(D, N))
    Dp, bias = r(D), 0.2 * r(D)
    steps = [dict(x=r(B, D, dt=bf), dt=(0.5 * r(B, D) - 1.0).to(bf), z=r(B, D, dt=bf),
                  B=r(B, N, dt=bf), C=r(B, N, dt=bf)) for _ in range(S)]

    def run_steps():
        return [selective_state_update(state, s_["x"], s_["dt"], A, s_["B"], s_["C"], Dp,
                                       s_["z"], bias, True) for s_ in steps]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_steps()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_steps()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    K = args.steps
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(K):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us_step = (time.perf_counter() - t0) * 1e6 / (K * S)
    ev_us = e0.elapsed_time(e1) * 1e3 / (K * S)
    # bytes per step, each tensor once: state read + written (fp32), A (fp32), x, dt, z, out
    # (bf16), B, C (bf16), D, dt_bias (fp32)
    nbytes = B * D * N * 4 * 2 + D * N * 4 + 4 * B * D * 2 + 2 * B * N * 2 + 2 * D * 4
    achieved = nbytes / (ev_us * 1e-6) / 1e9
    res = {
        "metric": "selective_state_update decode step latency (us per step) at 1 GPU",
        "value": round(us_step, 3), "unit": "us/step", "n_gpus": 1, "steps": K * S,
        "warmup": args.warmup, "ms_per_step": round(us_step / 1e3, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded normal inputs)",
        "config": {"workload": (f"decode: selective_state_update, batch {B}, dim {D}, dstate "
                                f"{N}, fp32 state, bf16 x/dt/z/B/C, softplus + dt_bias + D + z; "
                                f"{S} steps per HIP graph")},
        "gpu_event_us_per_step": round(ev_us, 3),
        "roofline": {"kernel": "ssu_rows_kernel (one per step, graph-launched)", "bound": "hbm",
                     "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": None,
                     "kernel_us_incl_graph_gaps": round(ev_us, 3),
                     "cache_resident": True,
                     "note": (f"the {B * D * N * 4 / 1e6:.1f} MB fp32 state stays in the 256 MB "
                              "Infinity Cache across the graph-replayed steps, so this rate is "
                              "cache bandwidth plus launch gaps, not HBM bandwidth")},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        from oracle.selective_state_update_ref import selective_state_update_ref
        torch.set_num_threads(os.cpu_count() or 1)
        st = state.cpu()
        cs = [{k: v.cpu() for k, v in s_.items()} for s_ in steps]
        Ac, Dc, bc = A.cpu(), Dp.cpu(), bias.cpu()
        ts = []
        for _ in range(3):
            t = time.perf_counter()
            for s_ in cs:
                selective_state_update_ref(st, s_["x"], s_["dt"], Ac, s_["B"], s_["C"], Dc,
                                           s_["z"], bc, True)
            ts.append((time.perf_counter() - t) * 1e6 / S)
        res["cpu_baseline"] = {"value": round(statistics.median(ts), 3), "unit": "us/step",
                               "cores": torch.get_num_threads(), "kind": "port", "cpu_model": cpu_model(),
                               "sample": f"restated selective_state_update_ref, the full "
                                         f"workload ({S} steps, median of 3 runs)"}
    print(json.dumps(res), flush=True)


SSD2 = dict(batch=8, seqlen=8192, nheads=24, headdim=64, ngroups=1, dstate=128, chunk=256)


def ssd_bytes(c, backward):
    """HBM bytes of the SSD path, each tensor once (bf16 activations): x, dt, B, C read and
    out written; the backward also reads dout and writes dx, ddt, dB, dC."""
    B, L, H, P, G, N = c["batch"], c["seqlen"], c["nheads"], c["headdim"], c["ngroups"], c["dstate"]
    fwd = 2 * (2 * B * L * H * P + B * L * H + 2 * B * L * G * N)
    if not backward:
        return fwd
    return fwd + 2 * (2 * B * L * H * P + B * L * H + 2 * B * L * G * N)


def ssd_flops(c):
    """Forward MFMA flops: chunk states and the entering-state term (2 B L H P N each), the
    intra-chunk product (2 B L H P Q / 2 on average, causal) and C B^T (B L G Q N)."""
    B, L, H, P, G, N, Q = (c["batch"], c["seqlen"], c["nheads"], c["headdim"], c["ngroups"],
                           c["dstate"], c["chunk"])
    return 4 * B * L * H * P * N + B * L * H * P * Q + B * L * G * Q * N


def ssd_scan_bytes(c):
    """Algorithmic HBM bytes of one ssd_chunk_scan launch, each tensor once: x read and out
    written (bf16), C (bf16), the passed states (bf16, one per chunk and head), the
    lower-triangle 64x64 tiles of C B^T (fp32) and the processed dt and cumsums (fp32)."""
    B, L, H, P, G, N, Q = (c["batch"], c["seqlen"], c["nheads"], c["headdim"], c["ngroups"],
                           c["dstate"], c["chunk"])
    K, qt = -(-L // Q), Q // 64
    return (2 * B * L * H * P * 2 + B * L * G * N * 2 + B * K * H * P * N * 2
            + B * K * G * (qt * (qt + 1) // 2) * 64 * 64 * 4 + 2 * B * H * K * Q * 4)


def run_ssd(torch, args):
    """Workload ssd2: Mamba-2's default SSD layer (headdim 64, dstate 128, chunk 256, one
    group, D per head, dt bias + softplus, no z: the RMSNorm variant, mamba2.py:30-56,
    209-225) at 24 heads (d_model 768), batch 8, seqlen 8192, bf16: one forward and one
    forward + backward of mamba_chunk_scan_combined."""
    from s6scan.ssd_combined import mamba_chunk_scan_combined, ssd_forward
    c = SSD2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, L, H, P, G, N, Q = (c["batch"], c["seqlen"], c["nheads"], c["headdim"], c["ngroups"],
                           c["dstate"], c["chunk"])
    g = torch.Generator("cpu").manual_seed(3)
    bf = torch.bfloat16
    r = lambda *s: torch.randn(*s, generator=g)
    sets = []
    for _ in range(2):
        sets.append(dict(x=r(B, L, H, P).to(dev, bf), dt=(0.5 * r(B, L, H) - 2.0).to(dev, bf),
                         B=r(B, L, G, N).to(dev, bf), C=r(B, L, G, N).to(dev, bf),
                         dy=r(B, L, H, P).to(dev, bf)))
    A = (-torch.exp(torch.rand(H, generator=g) * 2.77)).to(dev).requires_grad_(True)
    D = torch.randn(H, generator=g).to(dev).requires_grad_(True)
    bias = (0.3 * torch.randn(H, generator=g)).to(dev).requires_grad_(True)

    def fwd(i, ev=None):  # the forward launch sequence mamba_chunk_scan_combined runs
        s_ = sets[i % 2]
        with torch.no_grad():
            ssd_forward(s_["x"], s_["dt"], A, s_["B"], s_["C"], Q, D=D, dt_bias=bias,
                        dt_softplus=True, kernel_events=ev)

    def fwdbwd(i):
        s_ = sets[i % 2]
        leaves = {k: s_[k].detach().requires_grad_(True) for k in ("x", "dt", "B", "C")}
        out = mamba_chunk_scan_combined(leaves["x"], leaves["dt"], A, leaves["B"], leaves["C"], Q,
                                        D=D, dt_bias=bias, dt_softplus=True)
        out.backward(s_["dy"])

    res_t = {}
    mk = lambda: torch.cuda.Event(enable_timing=True)
    evs = [(mk(), mk()) for _ in range(args.steps)]
    for e0, e1 in evs:  # create the events; the library re-records them around ssd_chunk_scan
        e0.record(), e1.record()
    for name, fn in (("fwd", fwd), ("fwdbwd", fwdbwd)):
        for i in range(args.warmup):
            fn(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            fn(i, evs[i]) if name == "fwd" else fn(i)
        torch.cuda.synchronize()
        res_t[name] = (time.perf_counter() - t0) * 1e3 / args.steps
    scan_ms = sum(e0.elapsed_time(e1) for e0, e1 in evs) / len(evs)
    scan_gbps = ssd_scan_bytes(c) / (scan_ms * 1e-3) / 1e9
    traffic = None  # HBM bytes per ssd_chunk_scan launch, from the committed rocprofv3 counters
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            prof = json.load(f).get("ssd2")
        if prof:
            traffic = round(prof["traffic_bytes_per_launch"])
    tokch = B * L * H * P
    fl = ssd_flops(c)
    res = {
        "metric": "Mamba-2 SSD (mamba_chunk_scan_combined) fwd+bwd Mtok·ch/s at 1 GPU",
        "value": round(tokch / (res_t["fwdbwd"] * 1e-3) / 1e6, 2), "unit": "Mtok·ch/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(res_t["fwdbwd"], 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded normal inputs, Mamba-2 A init range [-16, -1])",
        "config": {"workload": (f"ssd2: batch {B}, seqlen {L}, nheads {H}, headdim {P}, ngroups "
                                f"{G}, dstate {N}, chunk {Q}; D per head, dt bias + softplus, no z")},
        "fwd_ms": round(res_t["fwd"], 5),
        "fwd_mtok_ch_per_s": round(tokch / (res_t["fwd"] * 1e-3) / 1e6, 2),
        "fwd_achieved": {"hbm_GBps_io_only": round(ssd_bytes(c, False) / (res_t["fwd"] * 1e-3) / 1e9, 2),
                         "mfma_TFLOPs": round(fl / (res_t["fwd"] * 1e-3) / 1e12, 2)},
        "roofline": {"kernel": "ssd_chunk_scan", "bound": "hbm", "achieved": round(scan_gbps, 2),
                     "peak": 8000.0, "unit": "GB/s", "frac": round(scan_gbps / 8000.0, 5),
                     "traffic": traffic, "kernel_ms": round(scan_ms, 5),
                     "algorithmic_bytes": ssd_scan_bytes(c)},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        from oracle.ssd_ref import ssd_chunked_ref
        torch.set_num_threads(os.cpu_count() or 1)
        Ls = 2048
        s_ = sets[0]
        cpu = {k: s_[k][:1, :Ls].float().cpu() for k in ("x", "dt", "B", "C")}
        Ac, Dc, bc = A.detach().cpu(), D.detach().cpu(), bias.detach().cpu()
        call = lambda n: ssd_chunked_ref(cpu["x"][:, :n], cpu["dt"][:, :n], Ac, cpu["B"][:, :n],
                                         cpu["C"][:, :n], Q, D=Dc, dt_bias=bc, dt_softplus=True)
        call(Q)  # untimed: first-call allocation and thread-pool start-up
        reps, t = 0, time.perf_counter()
        while reps < 200 and (reps == 0 or time.perf_counter() - t < 10.0):
            call(Ls)
            reps += 1
        sec = time.perf_counter() - t
        res["cpu_baseline"] = {"value": round(reps * Ls * H * P / sec / 1e6, 4), "unit": "Mtok·ch/s",
                               "cores": torch.get_num_threads(), "kind": "port", "cpu_model": cpu_model(),
                               "sample": (f"restated reference chunked forward (ssd_chunked_ref, "
                                          f"fp32 torch ops), batch 1, seqlen {Ls}, {reps} calls: "
                                          f"{sec:.2f} s")}
    print(json.dumps(res), flush=True)


def copy_reference(torch, steps):
    """Plain device-to-device copy of a known size (1 GiB read + 1 GiB written per launch).
    Profiled with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, it gives the factor between those
    counters and true HBM bytes that the scan kernels' counter readings are scaled by."""
    n = 1 << 28  # fp32 elements = 1 GiB
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(max(steps, 1)):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"workload": "copyref", "bytes_read_per_launch": 4 * n,
                      "bytes_written_per_launch": 4 * n, "launches": max(steps, 1)}))


def measure_scan(torch, workload, steps, warmup, layout="channel_last"):
    """One of the scan workloads (fwd1, fwdbwd3, fwd2, fwdbwd4, mixer1): its bench dict,
    without the CPU baseline.  ``layout`` "l_contiguous" stores every [B, L, *] input as
    [B, *, L] (same shape, time axis contiguous), so that the [B, *, L] arguments the steps
    pass (``.mT``) are L-contiguous, as zoology's Mamba passes them (mamba.py:128-132,
    176-179)."""
    import ctypes

    from s6scan import _lib
    from s6scan.configs import CONFIGS, make_inputs
    from s6scan.selective_scan_interface import selective_scan_backward, selective_scan_forward

    cfg = {"fwd1": CONFIGS[1], "fwdbwd3": CONFIGS[3], "fwd2": CONFIGS[2],
           "fwdbwd4": CONFIGS[4], "mixer1": CONFIGS[1]}[workload]
    mixer = workload == "mixer1"
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    # Three independent input sets (rotated every step) exceed the 256 MB Infinity Cache.
    nsets = 3
    sets = []
    import dataclasses
    for s in range(nsets):
        cpu = make_inputs(dataclasses.replace(cfg, seed=cfg.seed + 1000 * s))
        st = {k: v.to(dev) for k, v in cpu.items()}
        if mixer:
            st.update(mixer_extras(torch, st, torch.Generator("cpu").manual_seed(77 + s)))
        if layout == "l_contiguous":
            st = {k: (v.mT.contiguous().mT if v.dim() == 3 else v) for k, v in st.items()}
        sets.append(st)
        del cpu
    L = sets[0]["x"].shape[1]
    B = sets[0]["x"].shape[0]
    nbytes = cfg.algorithmic_bytes(seqlen=L)
    if mixer:  # + z read, + the gated output written next to the pre-gate one
        nbytes += 2 * B * L * cfg.dim * sets[0]["x"].element_size()

    def step(i, ev=None, ev_b=None, ev_f=None):
        g = sets[i % nsets]
        a = (g["x"].mT, g["delta"].mT, g["A"], g["B"].mT, g["C"].mT)
        cu = g.get("cu_seqlens")
        if mixer:  # the SSMMixer S6 core as s6scan.ssm_mixer.ssm_mixer_scan issues it
            with torch.no_grad():
                selective_scan_forward(g["x"].mT, g["dt_raw"].mT, -torch.exp(g["A_log"]),
                                       g["B"].mT, g["C"].mT, D=g["D"], z=g["z"].mT,
                                       delta_softplus=True, want_ckpt=False, kernel_events=ev)
        elif not cfg.backward:
            with torch.no_grad():
                selective_scan_forward(*a, D=g["D"], cu_seqlens=cu, want_ckpt=False,
                                       want_last_state=True, kernel_events=ev)
        else:
            if ev_f is not None:
                ev_f[0].record()
            out, _, xck, _ = selective_scan_forward(*a, D=g["D"], cu_seqlens=cu, want_ckpt=True,
                                                    want_last_state=True, kernel_events=ev)
            if ev_f is not None:
                ev_f[1].record()
            selective_scan_backward(*a, g["D"], None, None, False, g["dy"].mT, xck, cu_seqlens=cu,
                                    kernel_events=ev_b)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()

    K = steps
    mk = lambda: torch.cuda.Event(enable_timing=True)
    evs = [(mk(), mk()) for _ in range(K)]
    evs_b = [(mk(), mk()) for _ in range(K)] if cfg.backward else [None] * K
    evs_f = [(mk(), mk()) for _ in range(K)] if cfg.backward else [None] * K
    stream = torch.cuda.current_stream()
    for pair in evs + [p for p in evs_b if p is not None]:
        for e in pair:
            e.record(stream)  # creates the underlying hipEvent_t; re-recorded by the library
    g0, g1 = mk(), mk()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    g0.record(stream)
    for i in range(K):
        step(i, evs[i], evs_b[i], evs_f[i])
    g1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    ms_step = wall * 1e3 / K
    gpu_ms_step = g0.elapsed_time(g1) / K
    k_ms = statistics.mean(a.elapsed_time(b) for a, b in evs)
    kb_ms = statistics.mean(a.elapsed_time(b) for a, b in evs_b) if cfg.backward else None
    # whole forward (every kernel of the forward call): the step itself for the forward-only
    # workloads, the events around the forward call for the fwd+bwd ones
    fwd_ms = (statistics.mean(a.elapsed_time(b) for a, b in evs_f) if cfg.backward
              else gpu_ms_step)

    value = nbytes / (ms_step * 1e-3) / 1e9
    fwd_bytes = cfg.algorithmic_bytes(seqlen=L, with_backward=False) if cfg.backward else nbytes
    # Dominant kernel: the scan/output pass of the forward (backward main kernel for the
    # fwd+bwd workloads); one launch processes every (token, channel) of the call.
    g0_ = sets[0]
    from s6scan.selective_scan_interface import forward_kernel
    z0 = g0_["z"].mT if mixer else None
    d0 = g0_["dt_raw"] if mixer else g0_["delta"]
    kind = forward_kernel(g0_["x"].mT, d0.mT, g0_["A"], g0_["B"].mT, g0_["C"].mT,
                          g0_["D"], z0, None, mixer, g0_.get("cu_seqlens"))
    fwd_kernel = {"single_pass": "fwd_lanes (single-pass forward)",
                  "chunked": "fwd_scan (output pass of the chunked forward)",
                  "chunked_rows": "fwd_scan (output pass of the chunked forward, 8-step row "
                                  "blocks)"}[kind]
    if cfg.backward:
        dom_name, dom_ms, dom_bytes = "bwd_scan", kb_ms, nbytes - fwd_bytes
    else:
        dom_name, dom_ms, dom_bytes = fwd_kernel, k_ms, fwd_bytes
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    # HBM bytes per launch of the dominant kernel and its VALU busy fraction, measured with
    # rocprofv3 (FETCH_SIZE / WRITE_SIZE scaled by a plain-copy calibration; SQ counters) and
    # committed under profiles/.
    traffic = valu_busy = fwd_traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            prof = json.load(f).get(workload if layout == "channel_last" else workload + "_lc")
        if prof:
            traffic = round(prof["traffic_bytes_per_launch"])
            valu_busy = round(prof["kernels"][prof["dominant_kernel"]]["valu_busy"], 3)
            if prof.get("forward_traffic_bytes") is not None:
                fwd_traffic = round(prof["forward_traffic_bytes"])
    prof_src = ("profiles/traffic.json: rocprofv3 --pmc of this workload (FETCH_SIZE, WRITE_SIZE "
                "scaled by the plain-copy calibration; SQ counters), committed, not measured in "
                "this run")
    res = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "io_dtype": str(cfg.dtype).replace("torch.", ""),
        "data": "synthetic (seeded normal/uniform inputs of the workload's shape; 3 rotating sets)",
        "config": {"workload": (f"{cfg.name}: SSMMixer S6 core (softplus, D skip, z gate fused; "
                                "B/C slices of x_proj output)" if mixer else
                                f"{cfg.name}: s6scan selective_scan_forward"
                                f"{' + selective_scan_backward' if cfg.backward else ''} (the "
                                "launches selective_scan_fn makes) on "
                                + ("channel-last [B, L, D] views" if layout == "channel_last"
                                   else "[B, D, L] L-contiguous tensors")),
                   "layout": layout,
                   "forward_kernel": fwd_kernel,
                   "batch": B, "seqlen": L, "dim": cfg.dim, "dstate": cfg.dstate,
                   "nseq": cfg.nseq, "algorithmic_bytes_per_step": nbytes},
        "hbm_frac": round(value / HBM_PEAK_GBS, 5),
        "mtok_ch_per_s": round(B * L * cfg.dim / (ms_step * 1e-3) / 1e6, 2),
        "gpu_event_ms_per_step": round(gpu_ms_step, 5),
        "roofline": {
            "kernel": dom_name,
            "bound": "hbm",
            "achieved": round(achieved, 3),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5),
            "traffic": traffic,
            "kernel_ms": round(dom_ms, 5),
            # The kernels are VALU-bound (exp + 4-5 FMA-class ops per state element, packed
            # FP32 disabled); this is the measured fraction of SIMD cycles issuing VALU work.
            "valu_busy": valu_busy,
            "traffic_source": prof_src,
        },
        # every kernel of the forward call together (for the chunked forward: summaries, carry
        # and output pass), against the forward's algorithmic bytes
        "whole_forward": {
            "gpu_ms": round(fwd_ms, 5),
            "achieved": round(fwd_bytes / (fwd_ms * 1e-3) / 1e9, 3),
            "unit": "GB/s",
            "frac": round(fwd_bytes / (fwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 5),
            "algorithmic_bytes": fwd_bytes,
            "traffic": fwd_traffic,
            "traffic_source": prof_src,
        },
    }
    if cfg.backward:
        # state checkpoints held from the forward to the backward: fp32 [B, ceil(L/8), D, N]
        # (the reference's kernel saves [B, D, ceil(L/2048), 2N] fp32 and recomputes within
        # each 2048-step chunk, selective_scan_interface.py:42-50)
        nck = -(-L // 8)
        res["activation_bytes_per_layer"] = {
            "x_ckpt": B * nck * cfg.dim * cfg.dstate * 4,
            "reference_x": B * cfg.dim * -(-L // 2048) * 2 * cfg.dstate * 4,
        }
    if cfg.backward:
        res["fwd_kernel_ms"] = round(k_ms, 5)
    return res


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the scan shards over batch/channels without "
              "communication, so run it per GPU.", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.workload == "copyref":
        copy_reference(torch, args.steps)
        return
    import s6scan
    if args.workload == "mamba3":
        run_mamba(torch, args)
        return
    if args.workload == "decode":
        run_decode(torch, args)
        return
    if args.workload == "ssd2":
        run_ssd(torch, args)
        return
    res = measure_scan(torch, args.workload, args.steps, args.warmup, args.layout)
    if args.workload == "fwd1" and not args.no_fwdbwd:
        # BASELINE's metric covers fwd and fwd+bwd: the training-shape fwd+bwd (config 3)
        # rides along, measured the same way; value stays the config-1 forward.
        log("fwd+bwd (config 3) ...")
        fb = measure_scan(torch, "fwdbwd3", max(10, args.steps // 2), max(3, args.warmup // 2),
                          args.layout)
        res["fwd_bwd"] = {k: fb[k] for k in ("value", "unit", "ms_per_step", "hbm_frac",
                                              "mtok_ch_per_s", "steps", "config", "roofline",
                                              "fwd_kernel_ms", "whole_forward",
                                              "activation_bytes_per_layer")}
        if not args.no_cpu_baseline:
            from s6scan.configs import CONFIGS, make_inputs
            log("cpu baseline (config 3 sample) ...")
            res["fwd_bwd"]["cpu_baseline"] = cpu_baseline(CONFIGS[3], make_inputs,
                                                          one_thread=False)
    if not args.no_cpu_baseline:
        from s6scan.configs import CONFIGS, make_inputs
        log("cpu baseline ...")
        cfg = {"fwd1": CONFIGS[1], "fwdbwd3": CONFIGS[3], "fwd2": CONFIGS[2],
               "fwdbwd4": CONFIGS[4], "mixer1": CONFIGS[1]}[args.workload]
        res["cpu_baseline"] = cpu_baseline(cfg, make_inputs, mixer=args.workload == "mixer1")
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
