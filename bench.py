#!/usr/bin/env python3
"""Benchmark of the MI355X einsum_ir backend (one GPU).

Prints ONE JSON line.  The headline `value` is the binary-contraction
throughput of BASELINE config 3 -- the large bf16 batched multi-mode
contraction  zakm,zbkn->zabmn  (z8 a64 m64 b64 n64 k1024, bf16 inputs, fp32
accumulate and output) -- in GFLOP/s, with inputs resident in HBM.  A "step"
is one execution of that contraction (one kernel launch).  The other configs
(permute abcd->dbca in GB/s, the fp32 contraction of config 1, the 4-layer
MLP tree of config 4) are reported under "extra".

Before the config-3 timing the same kernel runs untimed for about one second
so the GPU is at its steady clock; the timed region is exactly --steps
launches after --warmup untimed ones.

`roofline` is for the dominant kernel (the config-3 contraction kernel):
achieved = 2*C*M*N*K FLOP per launch / average launch duration, measured with
HIP events recorded on the stream the kernel is launched on; peak = MI355X
dense bf16 MFMA 2516.6 TFLOP/s.  `traffic` (HBM bytes per launch) comes from
the committed rocprofv3 --pmc summary under profiles/ when present.

`cpu_baseline` times the CPU restatement of the reference algorithm
(oracle/oracle.c: fused loops, OpenMP tasks, packed fp32 blocked GEMM) on a
bounded sample of the same workload on the host cores; torch.einsum on the
host (the comparator the reference's harnesses print) is timed on the same
sample under extra["cpu_torch_einsum_c3_slice"], next to a probe of the host
(CPU model, cores, whether libxsmm / OpenBLAS are installed) and CPU rows for
configs 1, 2, 4 and 5 (extra["cpu_rows"]).
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-mfma-ceiling", action="store_true",
                   help="skip the matrix-core rate and clock probe (einsum_ir_amd/bin/mfma_ceiling)")
    p.add_argument("--only", default="", help="comma list of configs to run (c1,c2,c3,c4,c5,mlp,nodes,samples)")
    p.add_argument("--samples", default="",
                   help="with samples: comma list of what to run (tccg and/or einsum_benchmark network names; "
                        "default all)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also time a plain 512 MiB device copy (reference for the PMC byte counters)")
    p.add_argument("--settle", type=float, default=1.0,
                   help="seconds of untimed launches before the timing of configs 3, 4 and 5 (GPU clock settling)")
    p.add_argument("--summarize", nargs="+", metavar="DIR",
                   help="print statistics of rocprofv3 CSV output directories (kernel durations and/or "
                        "counters) over each kernel's last --timed dispatches, then exit (no GPU use)")
    p.add_argument("--timed", type=int, default=20,
                   help="with --summarize: dispatches per kernel and grid that form the timed region")
    p.add_argument("--kernel-filter", default="",
                   help="with --summarize: only kernels whose name matches this regular expression")
    return p.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def settle_clocks(torch, fn, seconds=1.0):
    """Runs fn() untimed for about `seconds` so the GPU reaches its steady
    clock under this load before anything is measured (the first kernels of a
    fresh process otherwise run up to 10 % slower while the clock ramps)."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_launches(torch, stream, fn, steps, warmup, settle=0.0):
    """Optionally settles the clock (untimed), runs fn() warmup times untimed,
    then steps times between HIP events on `stream`; returns (total seconds by
    host clock, average seconds per launch by device events)."""
    if settle > 0.0:
        settle_clocks(torch, fn, settle)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return t1 - t0, start.elapsed_time(end) * 1e-3 / steps


def _read_csv(path):
    import csv
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def summarize_rocprof(dirs, timed, kernel_filter=""):
    """Statistics of rocprofv3 `--output-format csv` results, per kernel and
    grid size, over the last `timed` dispatches of each (bench.py's timed
    launches: every workload launches its kernels only for the clock settle,
    the warm-up and then the timed steps) and over all of them.  Kernel
    durations come from run_kernel_trace.csv; counters from
    run_counter_collection.csv.  FETCH_SIZE / WRITE_SIZE (KiB per dispatch)
    are scaled to bytes by what the same counter reads for the run's first
    plain device copy (bench.py --calibrate-copy: 512 MiB each way, before
    any workload; later copies, such as the 1 GiB one of the permute rows,
    are not the calibration)."""
    import glob
    import statistics
    pat = re.compile(kernel_filter) if kernel_filter else None
    out = []
    durations = {}
    counters = {}          # (kernel, grid) -> counter -> [values in dispatch order]
    first_id = {}          # (kernel, grid) -> first dispatch id
    for d in dirs:
        for path in sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)):
            for r in _read_csv(path):
                grid = int(r["Grid_Size"]) if "Grid_Size" in r else \
                    int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
                key = (r["Kernel_Name"], grid)
                durations.setdefault(key, []).append(
                    (int(r["Start_Timestamp"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3))
        for path in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
            per = {}          # (kernel, grid) -> counter -> dispatch id -> value (summed over rows)
            for r in _read_csv(path):
                by_id = per.setdefault((r["Kernel_Name"], int(r["Grid_Size"])), {}).setdefault(r["Counter_Name"], {})
                d = int(r["Dispatch_Id"])
                by_id[d] = by_id.get(d, 0.0) + float(r["Counter_Value"])
            for k, cs in per.items():
                for c, by_id in cs.items():
                    counters.setdefault(k, {})[c] = [by_id[i] for i in sorted(by_id)]
                    first_id[k] = min(first_id.get(k, min(by_id)), min(by_id))
    if durations:
        out.append(f"# kernel durations (us): the last {timed} dispatches of each kernel and grid, and all of them")
        out.append(f"{'timed_avg':>10} {'timed_min':>10} {'timed_max':>10} {'all_avg':>10} {'calls':>6} "
                   f"{'grid':>9}  kernel")
        rows = []
        for (name, grid), v in durations.items():
            if pat and not pat.search(name):
                continue
            v.sort()
            last = [x for _, x in v[-timed:]]
            rows.append((sum(x for _, x in v), name, grid, last, [x for _, x in v]))
        for _, name, grid, last, alld in sorted(rows, reverse=True)[:40]:
            out.append(f"{statistics.mean(last):10.2f} {min(last):10.2f} {max(last):10.2f} "
                       f"{statistics.mean(alld):10.2f} {len(alld):6d} {grid:9d}  {name[:160]}")
    if counters:
        scale = {}
        for c, expect_kib in (("FETCH_SIZE", 524288.0), ("WRITE_SIZE", 524288.0)):
            copies = [(first_id[(n, g)], vals) for (n, g), cs in counters.items() for cc, vals in cs.items()
                      if cc == c and "copyBuffer" in n]
            if copies:
                # the calibration's own dispatches come first (the copy kernel's
                # grid does not depend on the size, so later copies share the group)
                _, vals = min(copies, key=lambda x: x[0])
                vals = vals[:5]
                scale[c] = expect_kib / statistics.mean(vals)
                out.append(f"# calibration: the 512 MiB device copy reads {c} = {statistics.mean(vals):.0f} KiB "
                           f"per dispatch; {c} is scaled by {scale[c]:.4f}")
        out.append(f"# counters: mean per dispatch over the last {timed} dispatches of each kernel and grid")
        for (name, grid), cs in sorted(counters.items()):
            if pat and not pat.search(name):
                continue
            out.append(f"## {name[:160]}  grid {grid}  ({max(len(v) for v in cs.values())} dispatches)")
            for c, vals in sorted(cs.items()):
                out.append(f"{c}: {statistics.mean(vals[-timed:]):.1f}")
            rd = statistics.mean(cs["FETCH_SIZE"][-timed:]) * 1024 * scale.get("FETCH_SIZE", 1) if "FETCH_SIZE" in cs else None
            wr = statistics.mean(cs["WRITE_SIZE"][-timed:]) * 1024 * scale.get("WRITE_SIZE", 1) if "WRITE_SIZE" in cs else None
            if rd is not None:
                out.append(f"hbm_read_bytes_per_launch: {rd:.0f}")
            if wr is not None:
                out.append(f"hbm_write_bytes_per_launch: {wr:.0f}")
            if rd is not None and wr is not None:
                out.append(f"hbm_bytes_per_launch: {rd + wr:.0f}")
    return "\n".join(out)


def traffic_from_profile(name):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary (FETCH_SIZE /
    WRITE_SIZE in KiB, scaled by the copy-kernel calibration factor)."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    m = re.search(r"^hbm_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def bench_c3(torch, eir, stream, steps, warmup, settle=1.0):
    sizes = dict(z=8, a=64, m=64, b=64, n=64, k=1024)
    loops = eir.binary_loops("zakm,zbkn->zabmn", sizes)
    g = torch.Generator(device="cuda").manual_seed(3)
    n_in = 8 * 64 * 1024 * 64
    left = (torch.rand(n_in, device="cuda", generator=g) * 2 - 1).to(torch.bfloat16)
    right = (torch.rand(n_in, device="cuda", generator=g) * 2 - 1).to(torch.bfloat16)
    out = torch.empty(8 * 64 * 64 * 64 * 64, device="cuda", dtype=torch.float32)
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"],
                               dtype_left=eir.BF16, dtype_right=eir.BF16, dtype_comp=eir.FP32,
                               dtype_out=eir.FP32)
    flops = plan.flops
    fn = lambda: plan.execute(left, right, out, stream=stream)
    wall, per_launch = time_launches(torch, stream, fn, steps, warmup, settle=settle)
    res = dict(flops=flops, wall=wall, per_launch=per_launch, desc=plan.describe(), bytes=plan.bytes)
    plan.close()
    del left, right, out
    return res


def bench_c3_comparators(torch, stream, steps, warmup):
    """Reference points for config 3 from the same run: its FLOPs as one
    batched GEMM through torch.bmm (hipBLASLt; 8 x [4096 x 1024] x
    [1024 x 4096], bf16 in, fp32 out; operands contiguous, K-contiguous A and
    N-contiguous B, not config 3's layout), and the 537 MB fp32 output written
    alone (torch fill_, the store floor of any kernel of this shape)."""
    g = torch.Generator(device="cuda").manual_seed(33)
    a = (torch.rand(8, 4096, 1024, device="cuda", generator=g) * 2 - 1).to(torch.bfloat16)
    b = (torch.rand(8, 1024, 4096, device="cuda", generator=g) * 2 - 1).to(torch.bfloat16)
    o = torch.empty(8, 4096, 4096, device="cuda", dtype=torch.float32)
    flops = 2 * 8 * 4096 * 4096 * 1024
    res = {}
    try:
        _, per = time_launches(torch, stream, lambda: torch.bmm(a, b, out_dtype=torch.float32), steps, warmup,
                               settle=0.5)
        res["torch_bmm_bf16_fp32out"] = dict(us_per_launch=round(per * 1e6, 2),
                                             tflops=round(flops / per * 1e-12, 1),
                                             frac_bf16_peak=round(flops / per * 1e-12 / PEAK_BF16_TFLOPS, 4))
    except Exception as e:   # an older torch without out_dtype
        res["torch_bmm_bf16_fp32out"] = f"unavailable: {e}"
    _, per = time_launches(torch, stream, lambda: o.fill_(1.5), steps, warmup)
    res["fill_fp32_output_537MB"] = dict(us_per_launch=round(per * 1e6, 2),
                                         gbs=round(o.numel() * 4 / per * 1e-9, 1))
    del a, b, o
    return res


def bench_c2(torch, eir, stream, steps, warmup):
    sizes = dict(a=64, b=64, c=64, d=64)
    u = eir.unary_dims("abcd->dbca", sizes)
    g = torch.Generator(device="cuda").manual_seed(2)
    x = torch.rand(64 ** 4, device="cuda", generator=g) * 2 - 1
    y = torch.empty_like(x)
    plan = eir.PermutePlan(u["sizes"], u["strides_in"], u["strides_out"], dtype=eir.FP32, ktype=eir.COPY)
    fn = lambda: plan.execute(x, y, stream=stream)
    wall, per_launch = time_launches(torch, stream, fn, steps, warmup)
    res = dict(bytes=plan.bytes, wall=wall, per_launch=per_launch, desc=plan.describe())
    plan.close()
    return res


# launches timed per figure for the kernels of a few to a few tens of
# microseconds (configs 1 and 2, the 4-D permutes): the first launch after
# an idle stream starts tens of microseconds after its start event, which
# 20 launches of a 22 us kernel would count as 15 % of the time
SHORT_STEPS = 200

PERMUTES_4D = [
    ("abcd->dbca", (64, 64, 64, 64)), ("abcd->dbca", (16, 256, 256, 16)), ("abcd->dbca", (8, 512, 512, 8)),
    ("abcd->dcba", (32, 32, 128, 128)), ("abcd->acdb", (128, 16, 64, 128)), ("abcd->bdac", (36, 48, 36, 512)),
    ("abcd->cabd", (48, 36, 512, 36)),
]


# tensors larger than the 256 MB Infinity Cache (MALL) in front of HBM: every
# launch reads and writes HBM itself (128^4 elements: 1 GiB each way in fp32,
# 512 MiB in bf16)
PERMUTES_BEYOND_CACHE = [("abcd->dbca", (128, 128, 128, 128)),
                         # same unit-stride dim on both sides: the vector copy,
                         # the ceiling any permutation of these bytes meets
                         ("abcd->bacd", (128, 128, 128, 128))]


def bench_permutes_4d(torch, eir, stream, dtype="fp32", shapes=None, steps=SHORT_STEPS):
    """Config 2's permutation kind over other 4-D shapes (COPY, 16.8-31.9 M
    elements, unit-stride dims from 8 to 512 wide): GB/s per shape, bytes =
    read + write of every element (reference src/bench_unary.cpp:230-306).
    The shapes of PERMUTES_4D move 67-255 MB per launch (fp32), so part of a
    run of launches can be served by the Infinity Cache; PERMUTES_BEYOND_CACHE
    cannot."""
    shapes = PERMUTES_4D if shapes is None else shapes
    tdt, edt, esz = (torch.float32, eir.FP32, 4) if dtype == "fp32" else (torch.bfloat16, eir.BF16, 2)
    rows = []
    # one input and one output buffer for all shapes: every shape runs on
    # memory the process already uses (freshly mapped pages are slower for
    # the first hundreds of launches, which the timed region would catch)
    n_max = max(s[0] * s[1] * s[2] * s[3] for _, s in shapes)
    x_all = torch.rand(n_max, device="cuda").to(tdt)
    y_all = torch.empty_like(x_all)
    for expr, shape in shapes:
        sizes = dict(zip("abcd", shape))
        u = eir.unary_dims(expr, sizes)
        n = shape[0] * shape[1] * shape[2] * shape[3]
        x = x_all[:n]
        y = y_all[:n]
        plan = eir.PermutePlan(u["sizes"], u["strides_in"], u["strides_out"], dtype=edt, ktype=eir.COPY)
        _, per = time_launches(torch, stream, lambda: plan.execute(x, y, stream=stream), steps, min(20, steps))
        gbs = 2 * esz * n / per * 1e-9
        rows.append(dict(expr=expr, sizes=list(shape), gbs=round(gbs, 1), frac_hbm_peak=round(gbs / PEAK_HBM_GBS, 4),
                         us_per_launch=round(per * 1e6, 2), kernel=plan.describe().split(" dims")[0]))
        plan.close()
    del x_all, y_all
    return rows


def bench_c1(torch, eir, stream, steps, warmup):
    sizes = dict(a=32, b=16, c=32, d=16, k=32, l=16)
    loops = eir.binary_loops("abkl,cdkl->abcd", sizes)
    g = torch.Generator(device="cuda").manual_seed(1)
    left = torch.rand(512 * 512, device="cuda", generator=g) * 2 - 1
    right = torch.rand(512 * 512, device="cuda", generator=g) * 2 - 1
    out = torch.empty(512 * 512, device="cuda")
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"])
    fn = lambda: plan.execute(left, right, out, stream=stream)
    wall, per_launch = time_launches(torch, stream, fn, steps, warmup)
    res = dict(flops=plan.flops, wall=wall, per_launch=per_launch, desc=plan.describe())
    plan.close()
    return res


def bench_c4(torch, eir, stream, steps, warmup, settle=0.0):
    """the 4-layer MLP tree bi,ih,hj,jk,ko->bo through
    EinsumExpression (left-to-right path, intermediates in the HBM arena, all
    nodes on one stream)."""
    from einsum_ir_amd import host
    b, w = 4096, 2048
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(b * w, device="cuda", generator=g)
    ws = [torch.randn(w * w, device="cuda", generator=g) / (w ** 0.5) for _ in range(4)]
    out = torch.empty(b * w, device="cuda")
    sizes = dict(b=b, i=w, h=w, j=w, k=w, o=w)
    e = host.Expression("bi,ih,hj,jk,ko->bo", sizes, [(0, 1), (0, 3), (0, 2), (0, 1)], [x] + ws + [out],
                        stream=stream)
    flops = 4 * 2 * b * w * w
    wall, per_eval = time_launches(torch, stream, e.eval_async, steps, warmup, settle=settle)
    res = dict(flops=flops, wall=wall, per_launch=per_eval, num_ops=e.num_ops(), arena=e.arena_bytes())
    e.close()
    return res


def bench_c5(torch, eir, stream, steps, warmup, settle=0.0):
    """the committed random tensor network (~50 GFLOP) through
    EinsumExpression along its greedy path."""
    from einsum_ir_amd import host
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "c5_network.json")))
    expr, sizes, path = fx["expr"], fx["sizes"], [tuple(p) for p in fx["path"]]
    ins, out = expr.split("->")
    g = torch.Generator(device="cuda").manual_seed(5)
    numel = lambda t: int(__import__("math").prod(sizes[d] for d in t))
    tensors = [torch.rand(numel(t), device="cuda", generator=g) * 2 - 1 for t in ins.split(",")]
    tensors.append(torch.empty(numel(out), device="cuda"))
    e = host.Expression(expr, sizes, path, tensors, stream=stream)
    wall, per_eval = time_launches(torch, stream, e.eval_async, steps, warmup, settle=settle)
    res = dict(flops=fx["flops"], wall=wall, per_launch=per_eval, num_ops=e.num_ops())
    e.close()
    # the same tree replayed as a recorded HIP graph (needs a stream of its own)
    gs = torch.cuda.Stream()
    e = host.Expression(expr, sizes, path, tensors, stream=gs)
    _, res["per_launch_graph"] = time_launches(torch, gs, e.eval_graph_async, steps, warmup, settle=settle)
    e.close()
    return res


def _expression_rate(torch, stream, expr, sizes_arg, path_arg, steps, warmup, seed):
    """Builds an EinsumExpression of a sample workload (inputs from
    harness.scaled_randn), times eval_async; returns (num_ops, s per eval)."""
    from einsum_ir_amd import harness, host
    ins, out = harness._tensors(expr)
    sizes = harness._sizes(expr, sizes_arg)
    path = harness._parse_path(path_arg)
    data = harness.scaled_randn(torch, ins, out, sizes, seed, torch.float32)
    dout = torch.empty([sizes[d] for d in out], device="cuda", dtype=torch.float32)
    e = host.Expression(expr, sizes, path, data + [dout], stream=stream)
    if steps is None:
        # as many evaluations as fill about 0.1 s (3 to 50): a short tree
        # needs several in flight for the host to enqueue ahead of the GPU
        _, per = time_launches(torch, stream, e.eval_async, 1, warmup)
        steps, warmup = max(3, min(50, int(0.1 / max(per, 1e-6)))), 0
    _, per = time_launches(torch, stream, e.eval_async, steps, warmup)
    n = e.num_ops()
    e.close()
    return n, per


def bench_samples(torch, eir, stream, which=()):
    """The reference's sample workloads (tests/golden/einsum_samples.json):
    the 59 TCCG binary contractions and the four einsum_benchmark networks at
    full size, fp32, each through EinsumExpression along its recorded path.
    Rates use num_ops() (the reference harnesses' flop count)."""
    import math
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "einsum_samples.json")))
    pick = lambda name: not which or name in which
    rates = []
    for c in (fx["tccg"] if pick("tccg") else []):
        n, per = _expression_rate(torch, stream, c["expr"], c["sizes"], c["path"], 10, 2,
                                  sum(map(ord, c["expr"])))
        rates.append((n / per * 1e-9, c["expr"]))
    tccg = None
    if rates:
        gm = math.exp(sum(math.log(r) for r, _ in rates) / len(rates))
        lo, hi = min(rates), max(rates)
        tccg = dict(cases=len(rates), unit="GFLOP/s", geomean=round(gm, 1),
                    frac_fp32_peak_geomean=round(gm / (PEAK_FP32_TFLOPS * 1e3), 4),
                    min=[round(lo[0], 1), lo[1]], max=[round(hi[0], 1), hi[1]])
    nets = {}
    for name, c in fx["einsum_benchmark"].items():
        if not pick(name):
            continue
        n, per = _expression_rate(torch, stream, c["expr"], c["sizes"], c["path"], None, 1, 11)
        nets[name] = dict(gflop=round(n * 1e-9, 2), ms_per_eval=round(per * 1e3, 3),
                          value=round(n / per * 1e-9, 1), unit="GFLOP/s",
                          frac_fp32_peak=round(n / per * 1e-12 / PEAK_FP32_TFLOPS, 4))
    return tccg, nets


def bench_mlp(torch, eir, stream, steps, warmup):
    """The reference's bench_mlp tree (src/bench_mlp.cpp:85-307): 784-512-512-
    512-512-10 MLP on a batch of 18 x 64, built node by node, bias COPY first
    touch broadcast over the batch, ReLU last touch, weights locked into device
    copies.  Seeded weights (the reference loads a TorchScript model)."""
    from einsum_ir_amd import host
    sizes = {0: 18, 1: 64, 2: 8, 3: 98, 4: 8, 5: 64, 6: 8, 7: 64, 8: 8, 9: 64, 10: 8, 11: 64, 12: 10}
    aux = {0: 1, 1: 1, 4: 8, 5: 64, 6: 8, 7: 64, 8: 8, 9: 64, 10: 8, 11: 64, 12: 10}
    ids_w = [[4, 5, 2, 3], [6, 7, 4, 5], [8, 9, 6, 7], [10, 11, 8, 9], [12, 10, 11]]
    ids_h = [[0, 1, 4, 5], [0, 1, 6, 7], [0, 1, 8, 9], [0, 1, 10, 11], [0, 1, 12]]
    widths = [784, 512, 512, 512, 512, 10]
    g = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn(1152 * 784, device="cuda", generator=g)
    ws = [(torch.rand(fo * fi, device="cuda", generator=g) * 2 - 1) / fi ** 0.5 for fi, fo in zip(widths, widths[1:])]
    bs = [(torch.rand(fo, device="cuda", generator=g) * 2 - 1) / fi ** 0.5 for fi, fo in zip(widths, widths[1:])]
    out = torch.empty(1152 * 10, device="cuda")

    def build(s):
        nodes = host.Nodes(sizes, aux, stream=s)
        prev = nodes.add_leaf([0, 1, 2, 3], x)
        n_w = [nodes.add_leaf(i, w) for i, w in zip(ids_w, ws)]
        for layer in range(5):
            last = eir.RELU if layer < 4 else eir.UNDEFINED_KTYPE
            prev = nodes.add_binary(ids_h[layer], prev, n_w[layer], tensor=out if layer == 4 else None,
                                    aux=bs[layer], first=eir.COPY, main=eir.MADD, last=last)
        nodes.compile(prev)
        for n in n_w:
            nodes.store_and_lock_data(n)
        return nodes

    nodes = build(stream)
    flops = nodes.num_ops()
    wall, per_eval = time_launches(torch, stream, nodes.eval_async, steps, warmup)
    nodes.close()
    # the same tree replayed as a recorded HIP graph (needs a stream of its own)
    gs = torch.cuda.Stream()
    nodes = build(gs)
    _, per_eval_graph = time_launches(torch, gs, nodes.eval_graph_async, steps, warmup)
    nodes.close()
    return dict(flops=flops, wall=wall, per_launch=per_eval, per_launch_graph=per_eval_graph)


# single tree nodes timed alone, each the shape one kernel family was tuned on:
# (name, expression, sizes, what bounds it)
NODES = [
    # einsum_benchmark lm_batch's largest matrix-vector node (403 MB, HBM-bound)
    ("lm_batch_gemv_C128_M1_N65536_K11", "ck,ckn->cn", dict(c=128, k=11, n=65536), "hbm"),
    # einsum_benchmark MERA's root on the short-K panel kernel (its operands'
    # and output's layouts as the tree lays them out are einsum_ir_amd's own;
    # this is the plain [m][n] layout of the same sizes)
    ("mera_root_M177147_N243_K50", "mk,nk->mn", dict(m=177147, k=50, n=243), "mfma"),
    # the one-short-side kernel: MERA's M = 11, N = 415800, K = 24 node
    # (HBM-bound), and an output laid out [long][short] (short side 13,
    # unit-stride), written as one block per workgroup
    ("mera_skinny_M11_N415800_K24", "mk,nk->mn", dict(m=11, k=24, n=415800), "hbm"),
    ("skinny_block_store_M400000_N13_K24", "mk,nk->mn", dict(m=400000, k=24, n=13), "hbm"),
]


def bench_nodes(torch, eir, stream, steps, warmup):
    """Single contraction nodes timed alone (inputs resident, back-to-back
    launches): rate against the HBM peak (algorithmic bytes: inputs + output)
    or the fp32 MFMA peak (2 C M N K flops)."""
    rows = []
    for name, expr, sizes, bound in NODES:
        lp = eir.binary_loops(expr, sizes)
        plan = eir.ContractionPlan(lp["dim_types"], lp["sizes"], lp["strides_left"], lp["strides_right"],
                                   lp["strides_out"])
        ins, out = expr.split("->")
        numel = lambda t: int(__import__("math").prod(sizes[d] for d in t))
        l_t, r_t = ins.split(",")
        a = torch.rand(numel(l_t), device="cuda")
        b = torch.rand(numel(r_t), device="cuda")
        o = torch.empty(numel(out), device="cuda")
        _, per = time_launches(torch, stream, lambda: plan.execute(a, b, o, stream=stream), steps, warmup)
        byt = 4 * (numel(l_t) + numel(r_t) + numel(out))
        row = dict(node=name, expr=expr, sizes=sizes, us_per_launch=round(per * 1e6, 2), kernel=plan.describe(),
                   bytes_per_launch=byt, gbs=round(byt / per * 1e-9, 1), flops_per_launch=plan.flops,
                   gflops=round(plan.flops / per * 1e-9, 1))
        row["frac_peak"] = round(row["gbs"] / PEAK_HBM_GBS if bound == "hbm" else row["gflops"] / (PEAK_FP32_TFLOPS * 1e3), 4)
        row["bound"] = bound
        rows.append(row)
        plan.close()
        del a, b, o
    return rows


def cpu_baseline_c3():
    """CPU restatement of the reference algorithm on a bounded sample of config 3:
    one batch (z=1), a=16 of 64 (M = 16*64 = 1024), all of N = 4096 and K = 1024."""
    import numpy as np
    from oracle import py_oracle as orc
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
    sizes = dict(z=1, a=16, m=64, b=64, n=64, k=1024)
    import einsum_ir_amd as eir
    loops = eir.binary_loops("zakm,zbkn->zabmn", sizes)
    rng = np.random.default_rng(3)
    a = orc.bf16_to_f32(orc.f32_to_bf16(rng.uniform(-1, 1, 16 * 1024 * 64).astype(np.float32)))
    b = orc.bf16_to_f32(orc.f32_to_bf16(rng.uniform(-1, 1, 64 * 1024 * 64).astype(np.float32)))
    out = np.empty(16 * 64 * 64 * 64, dtype=np.float32)
    flops = 2 * 1024 * 4096 * 1024
    orc.contract_blocked(loops, a, b, out, num_threads=threads)   # warm-up
    reps, t = 0, 0.0
    while t < 10.0 and reps < 50:
        t0 = time.perf_counter()
        orc.contract_blocked(loops, a, b, out, num_threads=threads)
        t += time.perf_counter() - t0
        reps += 1
    return dict(value=round(flops * reps / t * 1e-9, 2), unit="GFLOP/s", cores=threads, kind="port",
                sample=f"config-3 slice z=1,a=16 (M=1024,N=4096,K=1024; {flops/1e9:.2f} GFLOP) x{reps}, "
                       "fp32 math on the bf16-rounded inputs (the reference has no bf16 path); "
                       "oracle/oracle.c oracle_contract_blocked, OpenMP")


def cpu_torch_einsum_c3(threads):
    """torch.einsum on the host (the comparator the reference harnesses print,
    reference src/bench_binary.cpp:62-87) on the same config-3 slice as
    cpu_baseline_c3, fp32 on the bf16-rounded inputs."""
    import torch
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(3)
    a = (torch.rand(1, 16, 1024, 64, generator=g) * 2 - 1).bfloat16().float()
    b = (torch.rand(1, 64, 1024, 64, generator=g) * 2 - 1).bfloat16().float()
    flops = 2 * 1024 * 4096 * 1024
    torch.einsum("zakm,zbkn->zabmn", a, b)   # warm-up
    reps, t = 0, 0.0
    while t < 5.0 and reps < 50:
        t0 = time.perf_counter()
        torch.einsum("zakm,zbkn->zabmn", a, b)
        t += time.perf_counter() - t0
        reps += 1
    return dict(value=round(flops * reps / t * 1e-9, 2), unit="GFLOP/s", cores=threads,
                sample=f"config-3 slice z=1,a=16 (M=1024,N=4096,K=1024) x{reps}, fp32, "
                       f"torch {torch.__version__} CPU ({'MKL' if torch.backends.mkl.is_available() else 'no MKL'})")


def _cpu_rate(fn, work, budget=3.0, max_reps=20):
    """Average rate of fn() on the host: work / seconds, after one warm-up."""
    fn()
    reps, t = 0, 0.0
    while t < budget and reps < max_reps:
        t0 = time.perf_counter()
        fn()
        t += time.perf_counter() - t0
        reps += 1
    return work * reps / t, reps


def cpu_rows(threads):
    """CPU rows beside the GPU rows of configs 1, 2, 4 and 5 (baseline only):
    the reference algorithm restated (oracle: blocked contraction on all
    cores, blocked permute on one thread as the reference runs it) where it
    exists, and torch on the host, which the reference's
    harnesses print next to einsum_ir (src/bench_binary.cpp:62-87,
    src/bench_unary.cpp:311-323, src/bench_expression.cpp:381-422).  Full
    config sizes, about 3 s of work per row."""
    import numpy as np
    import torch
    import einsum_ir_amd as eir
    from oracle import py_oracle as orc
    torch.set_num_threads(threads)
    rows = {}
    g = torch.Generator().manual_seed(1)
    # config 1
    sizes = dict(a=32, b=16, c=32, d=16, k=32, l=16)
    loops = eir.binary_loops("abkl,cdkl->abcd", sizes)
    a = (torch.rand(512 * 512, generator=g) * 2 - 1).numpy()
    b = (torch.rand(512 * 512, generator=g) * 2 - 1).numpy()
    o = np.empty(512 * 512, np.float32)
    fl = 2 * 512 ** 3
    r1, n1 = _cpu_rate(lambda: orc.contract_blocked(loops, a, b, o, num_threads=threads), fl)
    ta, tb = torch.from_numpy(a).view(32, 16, 32, 16), torch.from_numpy(b).view(32, 16, 32, 16)
    r2, n2 = _cpu_rate(lambda: torch.einsum("abkl,cdkl->abcd", ta, tb), fl)
    rows["c1"] = dict(unit="GFLOP/s", port=round(r1 * 1e-9, 1), torch=round(r2 * 1e-9, 1), reps=[n1, n2])
    # config 2
    u = eir.unary_dims("abcd->dbca", dict(a=64, b=64, c=64, d=64))
    x = (torch.rand(64 ** 4, generator=g) * 2 - 1).numpy()
    y = np.empty_like(x)
    by = 2 * 4 * 64 ** 4
    r1, n1 = _cpu_rate(lambda: orc.permute_blocked(u["sizes"], u["strides_in"], u["strides_out"], x, y), by)
    tx = torch.from_numpy(x).view(64, 64, 64, 64)
    r2, n2 = _cpu_rate(lambda: tx.permute(3, 1, 2, 0).contiguous(), by)
    # the reference runs its unary loop nest on one thread
    rows["c2"] = dict(unit="GB/s", port=round(r1 * 1e-9, 1), port_cores=1, torch=round(r2 * 1e-9, 1),
                      reps=[n1, n2])
    # config 4: the MLP tree along its path
    w = 2048
    xs = torch.randn(4096, w, generator=g)
    ws = [torch.randn(w, w, generator=g) / w ** 0.5 for _ in range(4)]

    def mlp():
        h = xs
        for m in ws:
            h = torch.einsum("bi,ih->bh", h, m)
        return h
    r2, n2 = _cpu_rate(mlp, 4 * 2 * 4096 * w * w, max_reps=5)
    rows["c4"] = dict(unit="GFLOP/s", torch=round(r2 * 1e-9, 1), reps=[n2])
    # config 5: the committed network along its path
    from einsum_ir_amd import harness
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "c5_network.json")))
    ins, out = harness._tensors(fx["expr"])
    ts = [torch.rand([fx["sizes"][d] for d in t], generator=g) * 2 - 1 for t in ins]
    r2, n2 = _cpu_rate(lambda: harness.torch_path_eval(torch, ins, out, fx["sizes"],
                                                       [tuple(p) for p in fx["path"]], ts),
                       fx["flops"], max_reps=5)
    rows["c5"] = dict(unit="GFLOP/s", torch=round(r2 * 1e-9, 1), reps=[n2])
    rows["cores"] = threads
    return rows


def cpu_host_probe():
    """CPU model, core count and whether the reference's CPU libraries
    (libxsmm, OpenBLAS) are installed on this host."""
    import ctypes.util
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return dict(cpu_model=model, nproc=os.cpu_count(),
                libxsmm=ctypes.util.find_library("xsmm"), openblas=ctypes.util.find_library("openblas"))


def mfma_ceiling():
    """Runs einsum_ir_amd/bin/mfma_ceiling as a child process: the rate of an
    MFMA-only loop on every CU and the median shader clock of its waves, with
    constant and with random operands (the second is the power-limited clock
    that real data sees).  Returns {"<mfma>_<operands>": {...}}."""
    import subprocess
    exe = os.path.join(ROOT, "einsum_ir_amd", "bin", "mfma_ceiling")
    if not os.path.exists(exe):
        return {"error": "einsum_ir_amd/bin/mfma_ceiling is not built"}
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    if r.returncode != 0:
        return {"error": (r.stderr or r.stdout).strip()[-300:]}
    res = {}
    for ln in r.stdout.splitlines():
        if ln.startswith("{"):
            x = json.loads(ln)
            res[f"{x['mfma']}_{x['operands']}"] = {k: x[k] for k in ("tflops", "frac_peak", "clock_ghz_median")}
    return res


def main():
    args = parse_args()
    if args.summarize:
        print(summarize_rocprof(args.summarize, args.timed, args.kernel_filter))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU path. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    import einsum_ir_amd as eir
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    only = set(x for x in args.only.split(",") if x)
    run = lambda name: (not only) or (name in only)

    extra = {}
    c3 = None
    if args.calibrate_copy:
        n = 128 * 2 ** 20   # 512 MiB of fp32
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        wall, per = time_launches(torch, stream, lambda: dst.copy_(src), 5, 2)
        extra["copy_512MiB"] = dict(value=round(2 * 4 * n / per * 1e-9, 1), unit="GB/s",
                                    us_per_launch=round(per * 1e6, 2), bytes_per_launch=2 * 4 * n)
        log(f"copy: {per*1e6:.1f} us, {2 * 4 * n / per * 1e-9:.0f} GB/s")
        del src, dst
    if run("c3"):
        c3 = bench_c3(torch, eir, stream, args.steps, args.warmup, settle=args.settle)
        log(f"c3: {c3['desc']}  {c3['per_launch']*1e6:.1f} us/launch")
        extra["c3_reference_points"] = bench_c3_comparators(torch, stream, args.steps, args.warmup)
        log(f"c3 reference points: {extra['c3_reference_points']}")
    if run("c2"):
        c2 = bench_c2(torch, eir, stream, max(args.steps, SHORT_STEPS), args.warmup)
        gbs = c2["bytes"] / c2["per_launch"] * 1e-9
        extra["c2_permute_abcd_dbca_64^4_fp32"] = dict(
            value=round(gbs, 1), unit="GB/s", us_per_launch=round(c2["per_launch"] * 1e6, 2),
            frac_hbm_peak=round(gbs / PEAK_HBM_GBS, 4), bytes_per_launch=c2["bytes"], kernel=c2["desc"])
        log(f"c2: {c2['desc']}  {c2['per_launch']*1e6:.2f} us/launch  {gbs:.0f} GB/s")
        p4 = bench_permutes_4d(torch, eir, stream)
        extra["permutes_4d_fp32"] = dict(unit="GB/s", min_frac_hbm_peak=min(r["frac_hbm_peak"] for r in p4),
                                         cases=p4)
        log("permutes 4-D: " + ", ".join(f"{r['expr']}{r['sizes']} {r['gbs']:.0f}" for r in p4))
        p4b = bench_permutes_4d(torch, eir, stream, dtype="bf16")
        extra["permutes_4d_bf16"] = dict(unit="GB/s", min_frac_hbm_peak=min(r["frac_hbm_peak"] for r in p4b),
                                         cases=p4b)
        log("permutes 4-D bf16: " + ", ".join(f"{r['expr']}{r['sizes']} {r['gbs']:.0f}" for r in p4b))
        big = [dict(r, dtype=dt) for dt in ("fp32", "bf16")
               for r in bench_permutes_4d(torch, eir, stream, dtype=dt, shapes=PERMUTES_BEYOND_CACHE, steps=20)]
        # torch's copy of the same 1 GiB: the device's own read + write rate
        src = torch.rand(128 ** 4, device="cuda")
        dst = torch.empty_like(src)
        _, per = time_launches(torch, stream, lambda: dst.copy_(src), 20, 5)
        del src, dst
        torch_copy = round(2 * 4 * 128 ** 4 / per * 1e-9, 1)
        extra["permutes_beyond_infinity_cache"] = dict(
            unit="GB/s", note="tensors larger than the 256 MB Infinity Cache: HBM-resident every launch",
            torch_copy_1GiB_fp32_gbs=torch_copy, torch_copy_frac_hbm_peak=round(torch_copy / PEAK_HBM_GBS, 4),
            cases=big)
        log("permutes beyond the Infinity Cache: "
            + ", ".join(f"{r['dtype']} {r['expr']}{r['sizes']} {r['gbs']:.0f}" for r in big))
    if run("c1"):
        c1 = bench_c1(torch, eir, stream, max(args.steps, SHORT_STEPS), args.warmup)
        gf = c1["flops"] / c1["per_launch"] * 1e-9
        extra["c1_abkl_cdkl_fp32"] = dict(value=round(gf, 1), unit="GFLOP/s",
                                          us_per_launch=round(c1["per_launch"] * 1e6, 2),
                                          frac_fp32_peak=round(gf / (PEAK_FP32_TFLOPS * 1e3), 4),
                                          kernel=c1["desc"])
        log(f"c1: {c1['desc']}  {c1['per_launch']*1e6:.2f} us/launch")
    if run("nodes"):
        nodes = bench_nodes(torch, eir, stream, max(args.steps, 50), args.warmup)
        extra["single_nodes"] = nodes
        log("nodes: " + ", ".join(f"{r['node']} {r['us_per_launch']:.1f} us ({r['frac_peak']*100:.1f} % of the "
                                  f"{r['bound']} peak)" for r in nodes))
    if run("c4"):
        c4 = bench_c4(torch, eir, stream, max(5, args.steps // 5), min(args.warmup, 2), settle=args.settle)
        gf = c4["flops"] / c4["per_launch"] * 1e-9
        extra["c4_mlp_tree_fp32"] = dict(value=round(gf, 1), unit="GFLOP/s",
                                         ms_per_eval=round(c4["per_launch"] * 1e3, 3),
                                         frac_fp32_peak=round(gf / (PEAK_FP32_TFLOPS * 1e3), 4),
                                         path="EinsumExpression (4 contraction nodes, HBM arena "
                                              f"{c4['arena'] / 2**20:.0f} MiB)")
        log(f"c4: {c4['per_launch']*1e3:.3f} ms/eval")
    if run("c5"):
        c5 = bench_c5(torch, eir, stream, max(5, args.steps // 5), min(args.warmup, 2), settle=args.settle)
        gf = c5["flops"] / c5["per_launch"] * 1e-9
        extra["c5_tensor_network_fp32"] = dict(value=round(gf, 1), unit="GFLOP/s",
                                               ms_per_eval=round(c5["per_launch"] * 1e3, 3),
                                               frac_fp32_peak=round(gf / (PEAK_FP32_TFLOPS * 1e3), 4),
                                               flops_per_eval=c5["flops"],
                                               ms_per_eval_graph=round(c5["per_launch_graph"] * 1e3, 3),
                                               path="EinsumExpression, tests/golden/c5_network.json")
        log(f"c5: {c5['per_launch']*1e3:.3f} ms/eval, {c5['per_launch_graph']*1e3:.3f} ms/eval as graph replay")

    if run("mlp"):
        mlp = bench_mlp(torch, eir, stream, max(args.steps, 20), args.warmup)
        gf = mlp["flops"] / mlp["per_launch"] * 1e-9
        extra["bench_mlp_bias_relu_fp32"] = dict(value=round(gf, 1), unit="GFLOP/s",
                                                 us_per_eval=round(mlp["per_launch"] * 1e6, 2),
                                                 frac_fp32_peak=round(gf / (PEAK_FP32_TFLOPS * 1e3), 4),
                                                 flops_per_eval=mlp["flops"],
                                                 us_per_eval_graph=round(mlp["per_launch_graph"] * 1e6, 2),
                                                 path="EinsumNode tree, 5 contractions with bias COPY + ReLU, "
                                                      "weights locked")
        log(f"mlp: {mlp['per_launch']*1e6:.1f} us/eval, {mlp['per_launch_graph']*1e6:.1f} us/eval as graph replay")

    if run("samples"):
        tccg, nets = bench_samples(torch, eir, stream, set(x for x in args.samples.split(",") if x))
        if tccg is not None:
            extra["tccg_fp32"] = tccg
        extra["einsum_benchmark_fp32"] = nets
        log(f"tccg: {tccg}")
        for name, r in nets.items():
            log(f"{name}: {r}")

    if not args.no_mfma_ceiling and run("c3"):
        # after every GPU timing above: the probe runs the matrix cores flat out
        extra["mfma_ceiling"] = mfma_ceiling()
        log(f"mfma ceiling: {extra['mfma_ceiling']}")
        sustained = extra["mfma_ceiling"].get("bf16_32x32x16_random", {}).get("tflops")
        if c3 is not None and sustained:
            extra["c3_frac_sustained_bf16"] = round(c3["flops"] / c3["per_launch"] * 1e-12 / sustained, 4)

    cpu = None
    if not args.no_cpu_baseline and run("c3"):
        cpu = cpu_baseline_c3()
        log(f"cpu baseline: {cpu}")
        extra["cpu_torch_einsum_c3_slice"] = cpu_torch_einsum_c3(cpu["cores"])
        extra["cpu_host"] = cpu_host_probe()
        extra["cpu_rows"] = cpu_rows(cpu["cores"])
        log(f"cpu rows: {extra['cpu_rows']}")
        log(f"cpu torch.einsum: {extra['cpu_torch_einsum_c3_slice']}; host: {extra['cpu_host']}")

    if c3 is None:
        print(json.dumps({"extra": extra}))
        return
    value = c3["flops"] * args.steps / c3["wall"] * 1e-9
    achieved = c3["flops"] / c3["per_launch"] * 1e-12
    line = {
        "metric": "binary-contraction GFLOP/s & % MFMA peak; permute GB/s & % HBM peak (1 GPU)",
        "value": round(value, 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c3["wall"] / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform[-1,1], seeded torch generator, device-resident)",
        "config": {"workload": "zakm,zbkn->zabmn z=8 a=64 m=64 b=64 n=64 k=1024, bf16 in, fp32 acc+out "
                               "(BASELINE config 3)",
                   "C": 8, "M": 4096, "N": 4096, "K": 1024, "flops_per_step": c3["flops"],
                   "kernel": c3["desc"]},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profile("contract_bf16_c3_pmc.txt")},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
