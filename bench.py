"""MatRIS efsm throughput on one MI355X (atom.steps/s), with live kernel roofline numbers
and the CPU oracle timed on the host as a baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--c5-steps K5] [--no-c5] [--no-c2] [--no-c4]

`value`: a step is one full efsm evaluation of MatRIS-10M (num_layers=10, random init,
seed 0) on the C3 graph (864-atom fcc Cu): process_graphs, forward, torch.autograd.grad
for forces and stress, magmom head -- MatRIS.forward(graphs, task="efsm").  The graph
(built on the GPU once for the fixed C3 positions) is resident in HBM before the timed
region.

`c5_md`: the 32,000-atom a-SiO2 cell (C5) under NVT Berendsen MD (300 K, dt 1 fs,
tau 100 fs); every step rebuilds the radius and line graphs on the GPU from the new
positions and evaluates efs (forces for the integrator); interaction blocks are
checkpointed as far as the cell's activations exceed HBM.  40 of the config's 200 steps
by default (--c5-steps), after 2 warm-up steps.

`c4_batch`: the 64 random triclinic cells of C4 (8-64 atoms each) as one disjoint batch,
efsm, graphs built on the GPU once.

`captured` (C3, and inside `c4_batch`): the same evaluation replayed from a captured HIP
graph (MatRIS.capture, opt-in for graphs whose index arrays stay fixed), one status read
per replay.  `value` stays the eager rate.

`c2_line_attn`: the standalone line-attention core (forward, backward) and the
angle->bond segment sum on the C2 graph (4096-atom random packing) with N(0,1) features,
against HBM peak.

`roofline`: the dominant GatedMLP family (the most kernel time per step) against the MFMA
roofline of the arithmetic in use, its HBM figure alongside (`hbm`: the layer's inputs
and outputs, the saved pre-activations apart); `roofline_<other>`: the other direction;
`roofline_line_attn`: the line-attention forward against HBM; `hbm_in_model`: the HBM
fractions of the segment-sum, envelope-aggregation and line-attention families inside
the C3 step; `fp32_mfma`: the same C3 step with every GEMM in plain fp32 MFMA products.
Prints one JSON line.
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
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0
F16_MFMA_PEAK_TFLOPS = 2500.0
# The GEMM kernels compute each fp32 product as several 16-bit MFMA products (mma.h), so
# their ceiling in fp32-product terms is the dense 16-bit peak divided by that count.
# mode name -> (kernel template index, peak TFLOP/s in fp32 products, peak note, dtype)
MMA_ROOF = {
    "f16x3": (2, F16_MFMA_PEAK_TFLOPS / 3, "dense fp16 2500 TFLOP/s / 3 fp16 products per fp32 product",
              "fp32 (GEMMs: fp32 products as 3 fp16 MFMA products of an fp16 hi/lo split with a power-of-two "
              "weight scale, fp32 accumulate)"),
    "bf16x6": (6, BF16_MFMA_PEAK_TFLOPS / 6, "dense bf16 2500 TFLOP/s / 6 bf16 products per fp32 product",
               "fp32 (GEMMs: fp32 products as 6 bf16 MFMA products of an exact 3-way bf16 split, fp32 accumulate)"),
    "fp32": (0, FP32_MFMA_PEAK_TFLOPS, "dense fp32 MFMA 157.3 TFLOP/s", "fp32 (GEMMs: fp32 MFMA)"),
    "bf16x3": (3, BF16_MFMA_PEAK_TFLOPS / 3, "dense bf16 2500 TFLOP/s / 3 bf16 products per fp32 product",
               "fp32 in, ~2^-16 products (GEMMs: 2-way bf16 split, 3 MFMA products)"),
}
D = 128


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="C3", choices=["C3"])
    ap.add_argument("--c5-steps", type=int, default=40, help="timed C5 MD steps (after --c5-warmup)")
    ap.add_argument("--c5-warmup", type=int, default=2)
    ap.add_argument("--no-c5", action="store_true")
    ap.add_argument("--no-c2", action="store_true")
    ap.add_argument("--no-c4", action="store_true")
    ap.add_argument("--c5-only", action="store_true", help="run only the C5 MD line (for profiling)")
    ap.add_argument("--c4-only", action="store_true",
                    help="run only the C4 batch line, --steps timed evaluations after --warmup (for profiling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fp32-mfma", action="store_true", help="skip the plain fp32 MFMA (MODE 0) C3 step time")
    ap.add_argument("--cpu-sample-reps", type=int, default=6,
                    help="fcc reps of the CPU baseline sample (6: the C3 cell itself)")
    ap.add_argument("--cpu-steps", type=int, default=2, help="timed CPU baseline steps (after one warm-up)")
    ap.add_argument("--cpu-c5-proxy", action="store_true",
                    help="only time the CPU oracle on the reduced 4,000-atom a-SiO2 cell (no GPU)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="run one plain device copy of this many MiB first (HBM counter calibration)")
    return ap.parse_args()


def _captured_rate(model, graphs, n_atoms, steps, warmup):
    """atom*steps/s of MatRIS.capture(graphs) replays (each with its status read), over
    `steps` replays after `warmup`; the eager `value` stays the headline figure."""
    import torch
    cap = model.capture(graphs, task="efsm")
    for _ in range(warmup):
        cap.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        cap.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    del cap
    return dict(value=round(n_atoms * steps / dt, 2), unit="atom*steps/s", ms_per_step=round(dt / steps * 1e3, 3),
                steps=steps, warmup=warmup,
                note="opt-in HIP graph of the whole evaluation (MatRIS.capture): one replay and one status "
                     "read per step, for graphs whose index arrays stay fixed")


def _kernel_stats(timing):
    """Per kernel name: launches, mean duration (s), each launch's duration (ms) and the
    info records."""
    out = {}
    for name, evs in timing.items():
        ms = [a.elapsed_time(b) for a, b, _ in evs]
        out[name] = dict(n=len(ms), mean_s=sum(ms) / len(ms) / 1e3, ms=ms, info=[i for _, _, i in evs])
    return out


def _attn_line_bytes(A, U, with_perm=True):
    """Algorithmic HBM bytes of one line-attention forward launch: read alpha_t, alpha_s,
    e' [A,128] once, write y_t, y_s [E_u,128]; int32 source permutation and two int32
    row pointers.  The saved log-sum-exp statistics (2 x [E_u,128]) are reported apart."""
    return 4 * D * (3 * A + 2 * U) + (4 * A if with_perm else 0) + 8 * (U + 1)


def _gmlp_flops(M, K, tail_rows=0):
    """One fused GatedMLP forward (or backward, input gradients only):
    [M,K]x[K,256] plus two [M,128]x[128,128]; an FFN tail (forward) or head (backward) adds two
    more [M,128]x[128,128], the backward's pair projection one [M,256]x[256,128] (the same count)."""
    return 2.0 * M * (K * 256 + 2 * 128 * 128) + 2.0 * tail_rows * 2 * 128 * 128


# HBM bytes per launch measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by the
# 512 MiB copy calibration: x2.0 and x1.0) for the kernels the roofline fields describe,
# at C3 and at C2 (profiles/c3_efsm_hbm_traffic.md, which lists both).
# Keys: (launch name, config); a mean over that family's launches in one step where the
# shapes differ.
TRAFFIC_BYTES = {
    ("gmlp_bwd", "C3"): 559.8e6,       # every launch shape, 660 launches; at M = A 1129.8 MB (line attention,
                                       # plain instance) and 1525.8 MB (line refinement, with the FFN head)
    ("gmlp_fwd", "C3"): 588.6e6,       # every launch shape, 660 launches; at M = A 1483.7 MB (line attention,
                                       # with the logit projections) and 1339.6 MB (line refinement, with the FFN tail)
    ("attn_fwd_line", "C3"): 580.4e6,  # 537.9 read + 42.5 written
    ("attn_fwd", "C2"): 4061.9e6,
    ("attn_bwd", "C2"): 8461.9e6,
    ("seg_sum", "C2"): 1048.1e6,
}


def c4_batch(model, dev, steps: int, warmup: int):
    """Config C4: 64 random triclinic cells of 8-64 atoms (Z 1..94, seed 3) evaluated as one
    disjoint batch (efsm); graphs built on the GPU once, resident before the timed region."""
    import torch

    from matris_amd import workloads as W

    cells = W.c4_batch64()
    graphs = [model.graph_converter(c) for c in cells]
    n = sum(len(c) for c in cells)
    for _ in range(warmup):
        model(graphs, task="efsm")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model(graphs, task="efsm")
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    captured = _captured_rate(model, graphs, n, steps, warmup)
    return dict(metric="atom*steps/s (efsm of one disjoint batch of 64 cells)", value=round(n * steps / dt, 2),
                unit="atom*steps/s", steps=steps, warmup=warmup, ms_per_step=round(dt / steps * 1e3, 3),
                captured=captured,
                config={"workload": "C4: 64 random triclinic cells, 8-64 atoms, Z 1..94 (seed 3), one batch",
                        "n_atoms": n, "n_directed": sum(int(g.atom_graph.shape[0]) for g in graphs),
                        "n_angles": sum(int(g.line_graph.shape[0]) for g in graphs)})


def _events_time(fn, reps):
    """Mean seconds per call of fn, HIP events on torch's current stream (where every
    matris_hip launch goes)."""
    import torch
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps / 1e3


def c2_line_attn(dev, reps: int = 20):
    """Config C2 microbench: the line-attention core and the angle->bond segment sum on
    the 4096-atom random packing's line graph, features N(0,1) (seed 1, order
    alpha_s, alpha_t, e').  Algorithmic bytes count every input element read once and
    every output written once (int32 indices included); the gathered per-segment
    statistics of the backward are extra traffic, reported apart."""
    import torch

    from matris_amd import workloads as W
    from matris_amd.graph.converter import GraphConverter
    from matris_amd.model import ops

    cr = W.c2_rsa4096()
    g = GraphConverter(device=dev).from_arrays(cr.frac, cr.lattice, cr.z)
    lg = g.line_graph
    A, U = int(lg.shape[0]), int(g.undirected2directed.shape[0])
    tgt = ops.Grouping.build(lg[:, 1].contiguous(), U, sorted_rows=True)
    src = ops.Grouping.build(lg[:, 3].contiguous(), U)
    gen = torch.Generator().manual_seed(1)
    a_s, a_t, e = (torch.randn(A, D, generator=gen).to(dev) for _ in range(3))
    g_yt, g_ys = (torch.randn(U, D, generator=gen).to(dev) for _ in range(2))
    y_t, y_s, lse_t, lse_s = ops.attn_fwd_raw(a_t, a_s, e, tgt, src, None)
    t_f = _events_time(lambda: ops.attn_fwd_raw(a_t, a_s, e, tgt, src, None), reps)
    t_b = _events_time(lambda: ops.attn_bwd_raw(a_t, a_s, e, y_t, y_s, lse_t, lse_s, g_yt, g_ys, tgt, src, None),
                       reps)
    out = torch.empty(U, D, device=dev)
    t_s = _events_time(lambda: ops.seg_sum_raw(e, tgt, out=out), reps)
    b_f = 4 * D * (3 * A + 2 * U) + 4 * A + 8 * (U + 1)
    b_b = 4 * D * (6 * A + 2 * U) + 4 * A + 8 * (U + 1)
    b_s = 4 * D * (A + U) + 4 * A + 4 * (U + 1)

    def row(name, byts, t, key):
        gbs = byts / t / 1e9
        return dict(kernel=name, bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(gbs / HBM_PEAK_GBS, 4), traffic=TRAFFIC_BYTES.get((key, "C2")),
                    bytes_per_launch=byts, mean_us=round(t * 1e6, 2))

    return dict(workload="C2: 4096-atom random packing (rho 0.085, d_min 1.8, seed 1)", n_angles=A,
                n_undirected=U,
                fwd=row("attn_fwd_kernel<false>", b_f, t_f, "attn_fwd"),
                bwd=row("attn_bwd_kernel<false>", b_b, t_b, "attn_bwd") | dict(
                    extra_stat_bytes=4 * D * 4 * U, extra_stat_note="y_t, y_s, lse_t, lse_s gathered per row"),
                seg_sum=row("seg_sum_kernel", b_s, t_s, "seg_sum"))


def c5_md(model, dev, steps: int, warmup: int):
    """Config C5: NVT Berendsen MD of the 32,000-atom a-SiO2 cell, graph rebuilt on the
    GPU every step.  Returns atom.steps/s over `steps` steps after `warmup` steps."""
    import torch

    from matris_amd import workloads as W
    from matris_amd.applications.md import MolecularDynamics

    cr = W.c5_sio2_32k()
    torch.cuda.reset_peak_memory_stats(dev)
    md = MolecularDynamics((cr.frac, cr.lattice, cr.z), model=model, ensemble="nvt", thermostat="Berendsen",
                           temperature=300, starting_temperature=300, timestep=1.0, taut=100.0, task="efs",
                           device=str(dev), seed=4)
    md.run(warmup)
    torch.cuda.synchronize()
    md.timings = {"graph": 0.0, "model": 0.0}
    t0 = time.perf_counter()
    done = 0
    while done < steps:  # progress lines for long runs (each MD step ends in a stream sync anyway)
        k = min(20, steps - done)
        md.run(k)
        done += k
        print(f"c5 md: {done} of {steps} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    res = md.results
    from matris_amd.model import fused
    g = model.graph_converter(cr)  # after the timed region: the sizes behind the checkpoint choice
    n_ck = fused.blocks_to_checkpoint(int(g.line_graph.shape[0]), int(g.atom_graph.shape[0]),
                                      len(model.interaction_block), dev)
    del g
    return dict(
        metric="atom*steps/s (NVT MD step: GPU graph rebuild + efs fwd + autograd bwd + integrator)",
        value=round(len(cr) * steps / dt, 2), unit="atom*steps/s", steps=steps, warmup=warmup,
        ms_per_step=round(dt / steps * 1e3, 1),
        graph_ms_per_step=round(md.timings["graph"] / steps * 1e3, 2),
        model_ms_per_step=round(md.timings["model"] / steps * 1e3, 1),
        peak_mem_gib=round(torch.cuda.max_memory_allocated(dev) / 2 ** 30, 1),
        temperature_K=round(md.kinetic_temperature(), 2),
        e_per_atom=float(res["e"][0].detach()),
        config={"workload": "C5: 32,000-atom a-SiO2 (2.2 g/cm3, d_min 1.5, seed 4), NVT Berendsen 300 K, "
                            "dt 1 fs, tau 100 fs, MB velocities seed 4",
                "n_atoms": len(cr),
                "block_checkpoint": f"auto ({n_ck} of {len(model.interaction_block)} blocks)"})


def cpu_c5_proxy(steps: int, n_atoms: int = 4000):
    """The CPU oracle on a reduced a-SiO2 cell (BASELINE's C5 CPU plan: the 32,000-atom cell
    does not fit a CPU timing run, so the same generator at the same density with n_atoms
    atoms, seed 4), efs (forces and stress), one warm-up step then `steps` timed steps;
    atom-steps/s, labelled reduced."""
    import torch

    from matris_amd import workloads as W
    from matris_amd.config import MATRIS_10M
    from oracle import graph_ref
    from oracle.model_ref import MatRISRef

    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    cr = W.sio2(n_atoms, seed=4)
    og = graph_ref.build_graph(cr.frac, cr.lattice, cr.z)
    g = dict(atomic_number=torch.tensor(cr.z, dtype=torch.int32),
             atom_frac_coord=torch.tensor(cr.frac, dtype=torch.float32),
             lattice=torch.tensor(cr.lattice, dtype=torch.float32),
             neighbor_image=torch.tensor(og["image"], dtype=torch.float32),
             atom_graph=torch.tensor(np_stack(og["center"], og["neighbor"]), dtype=torch.int32),
             directed2undirected=torch.tensor(og["d2u"], dtype=torch.int32),
             undirected2directed=torch.tensor(og["u2d"], dtype=torch.int32),
             line_graph=torch.tensor(og["line_graph"], dtype=torch.int32))
    torch.manual_seed(0)
    model = MatRISRef(**MATRIS_10M).eval()
    print(f"cpu c5 proxy: {len(cr)} atoms, {len(og['line_graph'])} angles, {threads} threads", file=sys.stderr,
          flush=True)
    # a CPU evaluation of this cell runs for minutes: each interaction block reports when its
    # forward and its backward finish
    def report(i):
        def hook(_mod, _args, out):
            print(f"cpu c5 proxy: block {i} forward", file=sys.stderr, flush=True)
            if out[0].requires_grad:
                out[0].register_hook(lambda _g: print(f"cpu c5 proxy: block {i} backward", file=sys.stderr,
                                                      flush=True))
        return hook

    for i, blk in enumerate(model.interaction_block):
        blk.register_forward_hook(report(i))
    model([g], task="efs")
    t0 = time.perf_counter()
    for n in range(1, steps + 1):
        model([g], task="efs")
        print(f"cpu c5 proxy: step {n} of {steps} done", file=sys.stderr, flush=True)
    dt = time.perf_counter() - t0
    return dict(value=round(len(cr) * steps / dt, 3), unit="atom*steps/s", cores=threads, kind="port",
                sample=f"reduced: oracle/model_ref.py efs (fp32 torch CPU) on a {len(cr)}-atom a-SiO2 cell (2.2 g/cm3, "
                       f"d_min 1.5, seed 4; {len(og['center'])} edges, {len(og['line_graph'])} angles), {steps} timed "
                       f"steps after 1 warm-up, graph prebuilt")


def cpu_baseline(reps: int, steps: int):
    """The CPU oracle (oracle/model_ref.py, a plain fp32 torch restatement of the
    reference forward + autograd) on the host cores: the C3 cell itself at reps = 6 (a
    smaller fcc Cu reps^3 supercell with the same lattice constant and displacements
    otherwise), one warm-up step then `steps` timed steps.  Returns atom.steps/s and the
    thread count used (16: the GPU box's host share)."""
    import torch

    from matris_amd import workloads as W
    from matris_amd.config import MATRIS_10M
    from oracle import graph_ref
    from oracle.model_ref import MatRISRef

    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    cr = W.fcc_supercell(3.61, reps, sigma=0.05, seed=2)
    og = graph_ref.build_graph(cr.frac, cr.lattice, cr.z)
    g = dict(atomic_number=torch.tensor(cr.z, dtype=torch.int32),
             atom_frac_coord=torch.tensor(cr.frac, dtype=torch.float32),
             lattice=torch.tensor(cr.lattice, dtype=torch.float32),
             neighbor_image=torch.tensor(og["image"], dtype=torch.float32),
             atom_graph=torch.tensor(np_stack(og["center"], og["neighbor"]), dtype=torch.int32),
             directed2undirected=torch.tensor(og["d2u"], dtype=torch.int32),
             undirected2directed=torch.tensor(og["u2d"], dtype=torch.int32),
             line_graph=torch.tensor(og["line_graph"], dtype=torch.int32))
    torch.manual_seed(0)
    model = MatRISRef(**MATRIS_10M).eval()
    model([g], task="efsm")
    t0 = time.perf_counter()
    for n in range(1, steps + 1):
        model([g], task="efsm")
        print(f"cpu baseline: step {n} of {steps} done", file=sys.stderr, flush=True)
    dt = time.perf_counter() - t0
    return dict(value=round(len(cr) * n / dt, 3), unit="atom*steps/s", cores=threads, kind="port",
                sample=f"oracle/model_ref.py efsm (fp32 torch CPU) on fcc Cu {reps}x{reps}x{reps} "
                       f"({len(cr)} atoms, a=3.61, sigma=0.05 seed 2), {n} timed steps after 1 warm-up, "
                       f"graph prebuilt")


def np_stack(a, b):
    import numpy as np
    return np.stack([a, b], 1)


def main():
    args = _parse()
    if args.cpu_c5_proxy:
        print(json.dumps({"cpu_c5_proxy": cpu_c5_proxy(args.cpu_steps)}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested); multi-GPU scaling is a design "
              f"note, not built in this tree", file=sys.stderr)
        sys.exit(2)
    import torch

    from matris_amd import workloads as W
    from matris_amd.config import MATRIS_10M
    from matris_amd.model import MatRIS
    from matris_amd.model import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calib_copy_mib:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    torch.manual_seed(0)
    model = MatRIS(**MATRIS_10M).to(dev).eval()
    if args.c5_only:
        print(json.dumps({"c5_md": c5_md(model, dev, args.c5_steps, args.c5_warmup)}), flush=True)
        return
    if args.c4_only:
        print(json.dumps({"c4_batch": c4_batch(model, dev, args.steps, args.warmup)}), flush=True)
        return
    cr = W.c3_cu864()
    g = model.graph_converter(cr)
    n_atoms = len(cr)
    E_u = int(g.undirected2directed.shape[0])
    A = int(g.line_graph.shape[0])

    for _ in range(args.warmup):
        model([g], task="efsm")
    torch.cuda.synchronize()

    # per-kernel breakdown: a fully instrumented pass (an event pair around every launch of
    # this module) outside the timed region; it also names the dominant GatedMLP family
    timing_all = ops.enable_timing(True)
    n_brk = max(2, args.steps // 4)
    for _ in range(n_brk):
        model([g], task="efsm")
    torch.cuda.synchronize()
    ops.enable_timing(False)
    stats_all = _kernel_stats(timing_all)
    tot_all = {k: v["mean_s"] * v["n"] for k, v in stats_all.items()}
    dom = "gmlp_bwd" if tot_all.get("gmlp_bwd", 0) >= tot_all.get("gmlp_fwd", 0) else "gmlp_fwd"

    # timed region: HIP events only around the dominant kernel family's launches (events
    # around the other roofline kernels as well added ~0.3 ms to a 34 ms step)
    timing = ops.enable_timing(True, only=(dom,))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = model([g], task="efsm")
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ops.enable_timing(False)
    stats = _kernel_stats(timing)
    value = n_atoms * args.steps / dt

    # end-to-end including the GPU graph rebuild (the calculator's per-call path)
    t1 = time.perf_counter()
    e2e_steps = max(3, args.steps // 4)
    for _ in range(e2e_steps):
        gg = model.graph_converter(cr)
        model([gg], task="efsm")
    torch.cuda.synchronize()
    e2e = n_atoms * e2e_steps / (time.perf_counter() - t1)

    # the same step replayed from a captured HIP graph (opt-in; beside `value`)
    captured = _captured_rate(model, [g], n_atoms, args.steps, args.warmup)

    # rooflines: the dominant (MFMA-bound) kernel family and the line attention (HBM-bound)
    mode_idx, mma_peak, peak_note, dtype = MMA_ROOF[ops.get_mma_precision()]

    def gmlp_roof(name, st, n_steps, where):
        """The GatedMLP family against the MFMA roofline, the bound of the dense GEMMs on
        this path (kept fixed): achieved = algorithmic fp32-product FLOPs per
        launch / mean launch time, against the split-product peak of the arithmetic in use.
        The HBM figure rides along under `hbm`, its bytes the layer's inputs and outputs
        only (the pre-activations the build saves for its backward, p / z and the FFN's,
        are counted apart)."""
        gm = st.get(name)
        if not gm:
            return None
        info = gm["info"]
        flops = sum(_gmlp_flops(i["rows"], i["k"], i["extra_rows"]) for i in info) / gm["n"]
        byts_all = sum(i["bytes"] for i in info) / gm["n"]
        saved = sum(i["saved_bytes"] for i in info) / gm["n"]
        byts = byts_all - saved
        tf = flops / gm["mean_s"] / 1e12
        gbs = byts / gm["mean_s"] / 1e9
        n_line = sum(1 for i in info if i["rows"] == A)
        # every instance of the family: the Refinements' launches carry the FFN (forward tail /
        # backward head), the line attention's the logit projection pair (forward tail /
        # backward epilogue); MODE 6 runs the four-wave backward without a head or epilogue
        if name == "gmlp_fwd":
            kname = f"gmlp_fwd_kernel<{mode_idx}, *, *>"
        else:
            kname = f"gmlp_bwd_kernel<{mode_idx}>" if mode_idx == 6 else \
                f"gmlp_bwd8_kernel<{mode_idx}, *, *>"
        hbm = dict(achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=round(gbs / HBM_PEAK_GBS, 4),
                   bytes_per_launch=round(byts), saved_bytes_per_launch=round(saved),
                   achieved_with_saved=round(byts_all / gm["mean_s"] / 1e9, 1),
                   note="bytes: the layer's inputs (gathered sources as whole tables, projected sources as their "
                        "product tables, int32 indices, residual and gradient rows) read once and its outputs "
                        "written once; the saved pre-activations (p, z, the FFN's) apart, in "
                        "saved_bytes_per_launch and achieved_with_saved")
        return dict(bound="mfma", achieved=round(tf, 2), peak=round(mma_peak, 1), unit="TFLOP/s",
                    frac=round(tf / mma_peak, 4), traffic=TRAFFIC_BYTES.get((name, "C3")), kernel=kname,
                    mean_us=round(gm["mean_s"] * 1e6, 2), launches=gm["n"], flops_per_launch=round(flops),
                    frac_of_fp32_mfma_peak=round(tf / FP32_MFMA_PEAK_TFLOPS, 4), hbm=hbm,
                    note=f"means over {gm['n']} launches in {n_steps} steps of the {where} ({n_line} with "
                         f"M=A={A}); FLOPs 2*M*(256K+32768) with K the layer-1 width the kernel multiplies "
                         f"(+2*M*32768 for the launches that carry a Refinement's FFN or the line attention's "
                         f"pair projection), fp32 products; peak = {peak_note}")

    def inmodel_hbm(st, n_steps):
        """In-model HBM fractions of the reduction and attention families from the breakdown
        pass: algorithmic bytes (the byte formulas of the measurement plan: every input
        element read once, every output written once, int32 indices; saved statistics apart)
        summed over the family's launches / their summed duration; the angle-row (M = A)
        launches also on their own."""
        out = {}
        for fam in ("seg_sum", "env_agg_fwd", "env_agg_bwd", "attn_fwd_line", "attn_bwd_line"):
            v = st.get(fam)
            if not v:
                continue
            ms = v["ms"]
            info = v["info"]
            rows = [(i, t) for i, t in zip(info, ms) if isinstance(i, dict) and "bytes" in i]
            if not rows:
                continue

            def frac(sel):
                b = sum(i["bytes"] - i.get("saved_bytes", 0) for i, _ in sel)
                t = sum(t for _, t in sel) / 1e3
                gbs = b / t / 1e9
                return dict(achieved=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4), launches=len(sel),
                            bytes_per_step=round(b / n_steps), ms_per_step=round(t * 1e3 / n_steps, 3))
            out[fam] = dict(all=frac(rows))
            line = [(i, t) for i, t in rows if i.get("rows") == A]
            if line and len(line) != len(rows):
                out[fam]["angle_rows"] = frac(line)
        return dict(unit="GB/s", peak=HBM_PEAK_GBS, families=out,
                    note=f"HIP events around every launch of a {n_brk}-step breakdown pass (the event pair adds "
                         f"~1-2 us to each launch, so short launches read low)")

    other = "gmlp_fwd" if dom == "gmlp_bwd" else "gmlp_bwd"
    roof = gmlp_roof(dom, stats, args.steps, "timed region")
    r_other = gmlp_roof(other, stats_all, n_brk, "breakdown pass")
    at = stats_all.get("attn_fwd_line")
    attn = None
    hbm_inmodel = inmodel_hbm(stats_all, n_brk)
    if at:
        byts = _attn_line_bytes(A, E_u)
        gbs = byts / at["mean_s"] / 1e9
        attn = dict(kernel="attn_fwd_kernel<false>", bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS,
                    unit="GB/s", frac=round(gbs / HBM_PEAK_GBS, 4), traffic=TRAFFIC_BYTES.get(("attn_fwd_line", "C3")),
                    bytes_per_launch=byts,
                    mean_us=round(at["mean_s"] * 1e6, 2), launches=at["n"],
                    note=f"means over {at['n']} launches in {n_brk} steps of the breakdown pass")
    kern = {k: dict(launches=v["n"], mean_us=round(v["mean_s"] * 1e6, 2),
                    total_ms_per_step=round(v["mean_s"] * v["n"] * 1e3 / n_brk, 3)) for k, v in stats_all.items()}

    # the same step in plain fp32 MFMA products (MODE 0, v_mfma_f32_32x32x2f32) beside `value`
    fp32_mfma = None
    if not args.no_fp32_mfma:
        with ops.mma_precision("fp32"):
            for _ in range(2):
                model([g], task="efsm")
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            n32 = max(3, args.steps // 2)
            for _ in range(n32):
                model([g], task="efsm")
            torch.cuda.synchronize()
            dt32 = time.perf_counter() - t2
        fp32_mfma = dict(value=round(n_atoms * n32 / dt32, 2), unit="atom*steps/s",
                         ms_per_step=round(dt32 / n32 * 1e3, 3), steps=n32, warmup=2,
                         note="C3 efsm with every GEMM in plain fp32 MFMA products (mma_precision('fp32'), "
                              "v_mfma_f32_32x32x2f32) instead of the default f16x3 split")

    line = {
        "metric": "atom*steps/s (efsm fwd+autograd bwd), MatRIS-10M, 864-atom fcc Cu (C3)",
        "value": round(value, 2),
        "unit": "atom*steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (fcc Cu 6x6x6, sigma=0.05 A seed 2; random-init weights seed 0)",
        "config": {"workload": "C3: fcc Cu 6x6x6 conventional (864 atoms), efsm, MatRIS-10M (num_layers=10)",
                   "n_atoms": n_atoms, "n_directed": int(g.atom_graph.shape[0]), "n_undirected": E_u,
                   "n_angles": A,
                   "graph": "built on GPU once (fixed positions); its int32 index columns and CSR groupings are "
                            "built by the first evaluation and reused while its index tensors are unchanged; "
                            "geometry, strain and every layer run each step (e2e_with_gpu_graph_rebuild: the "
                            "radius graph, line graph and groupings rebuilt every step)"},
        "e2e_with_gpu_graph_rebuild": round(e2e, 2),
        "captured": captured,
        "roofline": roof,
        f"roofline_{other}": r_other,
        "roofline_line_attn": attn,
        "hbm_in_model": hbm_inmodel,
        "fp32_mfma": fp32_mfma,
        "kernels": kern,
        "kernels_note": f"per-launch HIP event timing of every kernel family over {n_brk} steps of a breakdown "
                        f"pass before the timed region (ms per step); inside the timed region only {dom} carries "
                        f"events (the `roofline` field); `roofline_{other}` and `roofline_line_attn` come from the "
                        f"breakdown pass",
        "e_per_atom": float(out["e"].item()),
    }
    if not args.no_c4:
        line["c4_batch"] = c4_batch(model, dev, max(3, args.steps // 2), 2)
    if not args.no_c2:
        line["c2_line_attn"] = c2_line_attn(dev)
    if not args.no_c5:
        line["c5_md"] = c5_md(model, dev, args.c5_steps, args.c5_warmup)
    if not args.no_cpu_baseline:
        try:
            line["cpu_baseline"] = cpu_baseline(args.cpu_sample_reps, args.cpu_steps)
        except Exception as exc:  # report, never fake
            line["cpu_baseline"] = dict(error=repr(exc))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
