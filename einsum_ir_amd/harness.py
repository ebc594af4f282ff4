"""Command-line harnesses of the reference, on the HIP backend.

    python -m einsum_ir_amd.harness binary     einsum_string dimension_sizes [dtype [loop_order]]
    python -m einsum_ir_amd.harness unary      einsum_string dimension_sizes [dtype]
    python -m einsum_ir_amd.harness expression einsum_string dimension_sizes contraction_path
                                               [dtype [store_lock [print_tree]]]
    python -m einsum_ir_amd.harness tree       einsum_tree dimension_sizes [dtype]

Arguments and printed reports follow the reference's bench_binary
(reference src/bench_binary.cpp:212-408), bench_unary (src/bench_unary.cpp:55-336),
bench_expression (src/bench_expression.cpp:8-545) and bench_tree
(src/bench_tree.cpp:8-173): dimension sizes in ascending order of the
dimension ids, dtypes FP32/FP64 (CPX_FP32/CPX_FP64 for expressions; BF16 is
additive), the same data generation (binary: left rand, right ones; unary:
rand; expression/tree: randn), the same FLOP and byte counts, the
"CSV_DATA:" lines, and a comparison with torch.einsum / torch.permute
(the reference compares with ATen).  Differences: tensors live on the GPU;
times are device times of the HIP stream (one warm-up, then repetitions for
~0.2 s; the reference times one evaluation on the host clock); the loop order
of bench_binary is accepted and ignored (one kernel grid runs every loop);
print_tree is not provided.
"""
import re
import sys
import time

from . import _lib
from . import host

_DT = {"FP32": _lib.FP32, "FP64": _lib.FP64, "BF16": _lib.BF16}


def _torch_dtype(torch, name):
    return {"FP32": torch.float32, "FP64": torch.float64, "BF16": torch.bfloat16,
            "CPX_FP32": torch.complex64, "CPX_FP64": torch.complex128}[name]


def _timed(torch, fn, min_seconds=0.2):
    """Device seconds per call: one warm-up, then repetitions for >= min_seconds."""
    fn()
    torch.cuda.synchronize()
    reps, total = 0, 0.0
    while total < min_seconds:
        n = max(1, reps)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        total += e0.elapsed_time(e1) * 1e-3
        reps += n
    return total / reps


def _tensors(expr):
    """Dim names of each tensor: single-character or bracketed standard format."""
    lhs, rhs = expr.replace(" ", "").split("->")
    if lhs.startswith("["):
        ins = [t.split(",") for t in re.findall(r"\[([^\[\]]*)\]", lhs)]
        out = rhs.strip("[]").split(",") if rhs.strip("[]") else []
    else:
        ins = [list(t) for t in lhs.split(",")]
        out = list(rhs)
    return ins, out


def _sizes(expr, sizes_arg):
    names = host.dim_names(expr)
    vals = [int(x) for x in sizes_arg.split(",") if x.strip()]
    if len(vals) != len(names):
        raise SystemExit(f"error: {len(names)} dimension sizes expected, got {len(vals)}")
    return dict(zip(names, vals))


def _print_parsed(ins, out, sizes):
    print("parsed tensors:")
    for t in ins + [out]:
        print("  " + ",".join(t))
    print("parsed dimension ids:")
    for i, n in enumerate(sizes):
        print(f"  {n}: {i}")
    print("parsed dimension sizes:")
    for n, s in sizes.items():
        print(f"  {n}: {s}")


def _torch_einsum(ins, out, sizes):
    letters = {}
    for n in sizes:
        letters[n] = chr(ord("a") + len(letters)) if len(letters) < 26 else chr(ord("A") + len(letters) - 26)
    return ",".join("".join(letters[d] for d in t) for t in ins) + "->" + "".join(letters[d] for d in out)


def _letters(dims):
    """Einsum letters for at most 52 distinct dims (torch.einsum's alphabet)."""
    m = {}
    for d in dims:
        if d not in m:
            n = len(m)
            m[d] = chr(ord("a") + n) if n < 26 else chr(ord("A") + n - 26)
    return m


def torch_pair(torch, da, a, db, b, dr):
    """One binary contraction a[da] * b[db] -> [dr] with torch.einsum, letters
    chosen per contraction so that expressions with more than 52 dims work."""
    m = _letters(list(da) + list(db))
    eq = "".join(m[d] for d in da) + "," + "".join(m[d] for d in db) + "->" + "".join(m[d] for d in dr)
    return torch.einsum(eq, a, b)


def torch_path_eval(torch, ins, out, sizes, path, data):
    """Evaluates an expression along its contraction path (opt_einsum's
    standard form: the pair is removed, the result appended) with torch.einsum
    in the dtype of `data`; intermediate dims are those still needed by the
    remaining tensors or the output."""
    ts = [(list(t), x) for t, x in zip(ins, data)]
    for i, j in path:
        (da, a), (db, b) = ts[i], ts[j]
        rest = [ts[k] for k in range(len(ts)) if k not in (i, j)]
        keep = set(out) | {d for t, _ in rest for d in t}
        dr = [d for d in dict.fromkeys(da + db) if d in keep]
        ts = rest + [(dr, torch_pair(torch, da, a, db, b, dr))]
    if len(ts) != 1:
        raise ValueError("contraction path does not reduce the expression to one tensor")
    dr, r = ts[0]
    return r.permute([dr.index(d) for d in out]) if dr != list(out) else r


def scaled_randn(torch, ins, out, sizes, seed, dtype):
    """N(0,1) inputs, tensor t scaled by prod(size of its contracted dims)^-1/4.
    A contracted dim of size s is shared by two tensors, so the products that
    its sum adds up have variance 1/s and the s-term sum variance 1: every
    contraction of a network keeps the values near unit magnitude (long
    networks leave the fp32 range otherwise)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    outs = set(out)
    data = []
    for t in ins:
        x = torch.randn([sizes[d] for d in t], device="cuda", dtype=torch.float64, generator=g)
        k = 1
        for d in t:
            if d not in outs:
                k *= sizes[d]
        data.append((x / k ** 0.25).to(dtype))
    return data


def _close(torch, ref, got, rtol=1e-3, atol=1e-4):
    ok = torch.allclose(ref.to(got.dtype), got, rtol=rtol, atol=atol)
    print("  results are close" if ok else f"  maximal difference is: {(ref.to(got.dtype) - got).abs().max().item()}")
    return ok


def bench_binary(argv):
    import torch
    print("running bench_binary!")
    expr, sizes_arg = argv[0], argv[1]
    dtype = argv[2] if len(argv) > 2 else "FP32"
    if dtype not in _DT:
        print("failed to determine dtype", file=sys.stderr)
        return 1
    ins, out = _tensors(expr)
    if len(ins) != 2:
        print("Einsum string is not a binary contraction", file=sys.stderr)
        return 1
    sizes = _sizes(expr, sizes_arg)
    _print_parsed(ins, out, sizes)
    print(f"dtype: {dtype}")
    if len(argv) > 3:
        print(f"loop order: {argv[3]} (ignored: the GPU plan runs every loop in one grid)")
    td = _torch_dtype(torch, dtype)
    shape = lambda t: [sizes[d] for d in t]
    left = torch.rand(shape(ins[0]), device="cuda").to(td)
    right = torch.ones(shape(ins[1]), device="cuda", dtype=td)
    outt = torch.rand(shape(out), device="cuda", dtype=torch.float32 if dtype == "BF16" else td)
    flops = 2
    for s in sizes.values():
        flops *= s
    eq = _torch_einsum(ins, out, sizes)
    t = _timed(torch, lambda: torch.einsum(eq, left.float() if dtype == "BF16" else left,
                                           right.float() if dtype == "BF16" else right))
    print("torch.einsum:")
    print(f"  time (contract): {t}")
    print(f"  gflops: {flops / t * 1e-9}")
    ref = torch.einsum(eq, left.double(), right.double())

    t0 = time.perf_counter()
    dl = _DT[dtype]
    b = host.Binary(expr, sizes, dtype_left=dl, dtype_right=dl, dtype_comp=_lib.FP64 if dtype == "FP64" else _lib.FP32,
                    dtype_out=_lib.FP64 if dtype == "FP64" else _lib.FP32)
    t_compile = time.perf_counter() - t0
    t = _timed(torch, lambda: b.contract(left, right, outt))
    print("einsum_ir:")
    print(f"  time (compile): {t_compile}")
    print(f"  time (contract): {t}")
    print(f"  gflops: {flops / t * 1e-9}")
    _close(torch, ref, outt, rtol=1e-2 if dtype == "BF16" else 1e-3)
    print(f"CSV_DATA: einsum_ir,\"{expr}\",\"{sizes_arg}\",{dtype},{flops},{t_compile},{t},{flops / t * 1e-9}")
    b.close()
    print("finished running bench_binary!")
    return 0


def bench_unary(argv):
    import torch
    expr, sizes_arg = argv[0].replace(" ", ""), argv[1]
    dtype = argv[2] if len(argv) > 2 else "FP32"
    if dtype not in _DT:
        print("failed to determine dtype", file=sys.stderr)
        return 1
    ins, out = _tensors(expr)
    sizes = _sizes(expr, sizes_arg)
    print("parsed tensors:")
    print("  " + "".join(ins[0]))
    print("  " + "".join(out))
    print("parsed dimension sizes:")
    for n, s in sizes.items():
        print(f"  {n}: {s}")
    print(f"dtype: {dtype}")
    td = _torch_dtype(torch, dtype)
    x = torch.rand([sizes[d] for d in ins[0]], device="cuda").to(td)
    y = torch.empty([sizes[d] for d in out], device="cuda", dtype=td)
    perm = [ins[0].index(d) for d in out]
    nbytes = 2 * x.numel() * x.element_size()
    print("total amount of transferred data (read + write):")
    print(f"  B:   {nbytes}")
    print(f"  MiB: {nbytes / 1024 ** 2}")
    print(f"  GiB: {nbytes / 1024 ** 3}")
    t0 = time.perf_counter()
    u = host.Unary(expr, sizes, dtype=_DT[dtype])
    t_compile = time.perf_counter() - t0
    t = _timed(torch, lambda: u.eval(x, y))
    print("einsum_ir:")
    print(f"  time (compile): {t_compile}")
    print(f"  time (eval):    {t}")
    print(f"  gibs (eval):    {nbytes / t / 1024 ** 3}")
    print(f"  gibs (total):   {nbytes / (t + t_compile) / 1024 ** 3}")
    tp = _timed(torch, lambda: x.permute(perm).contiguous())
    print("torch.permute:")
    print(f"  time (total):   {tp}")
    print(f"  gibs (total):   {nbytes / tp / 1024 ** 3}")
    ok = torch.equal(x.permute(perm).contiguous(), y)
    print("  results are equal" if ok else "  results differ")
    print(f"CSV_DATA: einsum_ir,\"{expr}\",\"{sizes_arg}\",{dtype},{nbytes},{t_compile},{t},{nbytes / t / 1024 ** 3}")
    u.close()
    return 0 if ok else 1


def _parse_path(path_arg):
    nums = [int(x) for x in re.findall(r"-?\d+", path_arg)]
    return [tuple(nums[i:i + 2]) for i in range(0, len(nums), 2)]


def bench_expression(argv):
    import torch
    expr, sizes_arg, path_arg = argv[0], argv[1], argv[2]
    dtype = argv[3] if len(argv) > 3 else "FP32"
    store_lock = len(argv) > 4 and argv[4] == "1"
    if len(argv) > 5 and argv[5] != "0":
        print("print_tree is not provided by this harness", file=sys.stderr)
    ctype = host.BATCH_INNER if dtype.startswith("CPX_") else host.REAL_ONLY
    base = dtype[4:] if ctype != host.REAL_ONLY else dtype
    if base not in ("FP32", "FP64"):
        print("failed to determine dtype", file=sys.stderr)
        return 1
    ins, out = _tensors(expr)
    sizes = _sizes(expr, sizes_arg)
    path = _parse_path(path_arg)
    _print_parsed(ins, out, sizes)
    print(f"parsed contraction path: {path}")
    print(f"dtype: {dtype}")
    td = _torch_dtype(torch, dtype)
    data = [torch.randn([sizes[d] for d in t], device="cuda", dtype=td) for t in ins]
    outt = torch.zeros([sizes[d] for d in out], device="cuda", dtype=td)
    t0 = time.perf_counter()
    e = host.Expression(expr, sizes, path, data + [outt], dtype=_DT[base], ctype=ctype)
    if store_lock:
        for i in range(len(ins) - 1):
            e.store_and_lock_data(i)
    t_compile = time.perf_counter() - t0
    t = _timed(torch, e.eval)
    flops = e.num_ops()
    print("einsum_ir:")
    print(f"  #flops:         {flops}")
    print(f"  time (compile): {t_compile}")
    print(f"  time (eval):    {t}")
    print(f"  gflops (eval):  {flops / t * 1e-9}")
    print(f"  gflops (total): {flops / (t + t_compile) * 1e-9}")
    print(f"CSV_DATA: einsum_ir,\"{expr}\",\"{sizes_arg}\",\"{path_arg}\",{flops},{t_compile},{t},"
          f"{flops / t * 1e-9},{flops / (t + t_compile) * 1e-9}")
    hi = torch.complex128 if ctype != host.REAL_ONLY else torch.float64
    if len(sizes) <= 52:
        eq = _torch_einsum(ins, out, sizes)
        ref = torch.einsum(eq, *[d.to(hi) for d in data])
        tt = _timed(torch, lambda: torch.einsum(eq, *data))
    else:
        # more dims than torch.einsum has letters: contract along the path
        ref = torch_path_eval(torch, ins, out, sizes, path, [d.to(hi) for d in data])
        tt = _timed(torch, lambda: torch_path_eval(torch, ins, out, sizes, path, data))
    print("torch.einsum:")
    print(f"  time (eval):    {tt}")
    print(f"  gflops (eval):  {flops / tt * 1e-9}")
    print(f"CSV_DATA: torch.einsum,\"{expr}\",\"{sizes_arg}\",\"{path_arg}\",{flops},0,{tt},{flops / tt * 1e-9},"
          f"{flops / tt * 1e-9}")
    ok = _close(torch, ref, outt)
    e.close()
    return 0 if ok else 1


def _parse_tree(s):
    """Bracketed tree format -> post-order list of (dims, children)."""
    nodes = []

    def dims_of(txt):
        return [int(x) for x in txt.split(",") if x]

    def parse(txt):
        # txt: "child,child->[dims]" or "child->[dims]" or a leaf "[dims]"
        depth, arrow = 0, -1
        for i, ch in enumerate(txt):
            if ch == "[":
                depth += 1
            elif ch == "]":
                depth -= 1
            elif ch == "-" and depth == 0 and txt[i + 1] == ">":
                arrow = i
        if arrow < 0:
            nodes.append((dims_of(txt.strip("[]")), []))
            return len(nodes) - 1
        lhs, rhs = txt[:arrow], txt[arrow + 2:]
        parts, depth, start = [], 0, 0
        for i, ch in enumerate(lhs):
            if ch == "[":
                depth += 1
            elif ch == "]":
                depth -= 1
            elif ch == "," and depth == 0:
                parts.append(lhs[start:i])
                start = i + 1
        parts.append(lhs[start:])
        kids = []
        for p in parts:
            inner = p[1:-1]
            kids.append(parse(inner) if "->" in inner else parse(p))
        nodes.append((dims_of(rhs.strip("[]")), kids))
        return len(nodes) - 1

    parse(s.replace(" ", ""))
    return nodes


def torch_tree_eval(torch, nodes, tensors, dtype):
    """Values of every node of a parsed tree (post-order list from
    _parse_tree), computed node by node with torch.einsum in `dtype`."""
    vals = []
    for (dims, kids), t_in in zip(nodes, tensors):
        if not kids:
            vals.append(t_in.to(dtype))
        elif len(kids) == 1:
            src = nodes[kids[0]][0]
            vals.append(vals[kids[0]].permute([src.index(d) for d in dims]))
        else:
            (da, db) = nodes[kids[0]][0], nodes[kids[1]][0]
            vals.append(torch_pair(torch, da, vals[kids[0]], db, vals[kids[1]], dims))
    return vals


def bench_tree(argv):
    import torch
    tree, sizes_arg = argv[0], argv[1]
    dtype = argv[2] if len(argv) > 2 else "FP32"
    if dtype not in ("FP32", "FP64"):
        print("failed to determine dtype", file=sys.stderr)
        return 1
    sizes = [int(x) for x in sizes_arg.split(",")]
    nodes = _parse_tree(tree)
    td = _torch_dtype(torch, dtype)
    tensors = []
    for dims, kids in nodes:
        if not kids:
            tensors.append(torch.randn([sizes[d] for d in dims], device="cuda", dtype=td))
        else:
            tensors.append(None)
    root = torch.zeros([sizes[d] for d in nodes[-1][0]], device="cuda", dtype=td)
    tensors[-1] = root
    t0 = time.perf_counter()
    tr = host.Tree(tree, sizes, tensors, dtype=_DT[dtype])
    t_compile = time.perf_counter() - t0
    t = _timed(torch, tr.eval)
    flops = tr.num_ops()
    print("einsum_ir:")
    print(f"  #flops:         {flops}")
    print(f"  time (compile): {t_compile}")
    print(f"  time (eval):    {t}")
    print(f"  gflops (eval):  {flops / t * 1e-9}")
    print(f"  gflops (total): {flops / (t + t_compile) * 1e-9}")
    print(f"CSV_DATA: einsum_ir,\"{tree}\",\"{sizes_arg}\",{flops},{t_compile},{t},{flops / t * 1e-9},"
          f"{flops / (t + t_compile) * 1e-9}")

    # reference: evaluate the tree with torch.einsum node by node in float64
    vals = torch_tree_eval(torch, nodes, tensors, torch.float64)
    ok = _close(torch, vals[-1], root)
    tr.close()
    return 0 if ok else 1


def main(argv=None):
    argv = list(sys.argv[1:] if argv is None else argv)
    cmds = {"binary": (bench_binary, 2), "unary": (bench_unary, 2), "expression": (bench_expression, 3),
            "tree": (bench_tree, 2)}
    if not argv or argv[0] not in cmds or len(argv) - 1 < cmds[argv[0]][1]:
        print(__doc__, file=sys.stderr)
        return 1
    fn, _ = cmds[argv[0]]
    return fn(argv[1:])


if __name__ == "__main__":
    sys.exit(main())
