"""Seeded randomized parity: binary contractions, permutations and trees drawn
at random (dimension roles and counts, sizes including 1 and ragged ones,
tensor layouts, dtypes, touch kernels), each checked against the CPU oracle
on identical inputs.  The draws cover the planner's paths (role swap, load
modes, affine and table K, tile choices, split K) without naming them.

Bars as everywhere: fp32 relative Frobenius <= 1e-5, bf16 inputs <= 2e-3,
fp64 <= 1e-12, permutations bit-exact.
"""
import string

import numpy as np
import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import host
from tests.helpers import TOL_BF16, TOL_FP32, rel_frobenius, tensor_numel
from tests.test_gpu_contract import run_case
from tests.test_gpu_permute import _check as permute_check

pytestmark = pytest.mark.gpu

SIZES = [1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 24, 31, 32, 48, 64, 65, 96, 128]


def _draw_sizes(rng, dims, budget):
    """Sizes for dims whose product stays at or below budget."""
    sizes = {}
    prod = 1
    for d in dims:
        cands = [s for s in SIZES if prod * s <= budget] or [1]
        s = int(rng.choice(cands))
        sizes[d] = s
        prod *= s
    return sizes


def _shrink(sizes, cost, budget):
    """Halves the largest size until cost(sizes) <= budget (the oracle's
    scalar loops must finish in well under a second per case)."""
    while cost(sizes) > budget:
        d = max(sizes, key=lambda x: sizes[x])
        sizes[d] = max(1, sizes[d] // 2 + (sizes[d] % 2 if sizes[d] > 2 else 0))
    return sizes


def _binary_case(seed):
    rng = np.random.default_rng(1000 + seed)
    letters = list(string.ascii_lowercase)
    rng.shuffle(letters)
    nc, nm, nn, nk = (int(rng.integers(0, 3)), int(rng.integers(1, 4)), int(rng.integers(1, 4)),
                      int(rng.integers(1, 4)))
    dims = letters[:nc + nm + nn + nk]
    c, m, n, k = dims[:nc], dims[nc:nc + nm], dims[nc + nm:nc + nm + nn], dims[nc + nm + nn:]
    long_k = seed % 7 == 0          # small M x N, long K: the split-K path
    sizes = {}
    sizes.update(_draw_sizes(rng, c, 16))
    sizes.update(_draw_sizes(rng, m, 128 if long_k else 2048))
    sizes.update(_draw_sizes(rng, n, 128 if long_k else 2048))
    sizes.update(_draw_sizes(rng, k, 16384 if long_k else 1024))
    _shrink(sizes, lambda s: int(np.prod(list(s.values()))), 1 << 25)
    left = list(rng.permutation(c + m + k))
    right = list(rng.permutation(c + n + k))
    out = list(rng.permutation(c + m + n))
    expr = "".join(left) + "," + "".join(right) + "->" + "".join(out)
    dtype = [eir.FP32, eir.FP32, eir.BF16, eir.FP64][seed % 4]
    first = [eir.ZERO, eir.COPY, eir.ADD, eir.UNDEFINED_KTYPE][int(rng.integers(0, 4))]
    last = [eir.UNDEFINED_KTYPE, eir.RELU, eir.ADD][int(rng.integers(0, 3))]
    dtype_out = eir.BF16 if dtype == eir.BF16 and seed % 8 == 2 else eir.FP32
    return expr, sizes, dtype, dtype_out, first, last


@pytest.mark.parametrize("seed", range(200))
def test_random_binary(torch_cuda, oracle, seed):
    expr, sizes, dtype, dtype_out, first, last = _binary_case(seed)
    print(f"random binary {seed}: {expr} {sizes} dtype {dtype}/{dtype_out} touch {first}/{last}", flush=True)
    run_case(torch_cuda, oracle, expr, sizes, dtype=dtype, first=first, last=last, seed=seed,
             dtype_out=dtype_out)


# tiles a test may force through the planner's diagnostic override; the
# planner ignores a forced tile that does not fit the contraction (dtype, load
# modes, alignment), and the case then runs its default
FORCE_TILES = {eir.FP32: [0, 1], eir.BF16: [2, 3, 4, 6, 7, 8]}


@pytest.mark.parametrize("seed", range(80))
def test_random_binary_forced_tile(torch_cuda, oracle, monkeypatch, seed):
    """Random contractions on every kernel instantiation, not only on the one
    the planner would choose for the shape."""
    expr, sizes, dtype, dtype_out, first, last = _binary_case(500 + seed)
    if dtype == eir.FP64:
        dtype = eir.BF16 if seed % 2 else eir.FP32
    tiles = FORCE_TILES[dtype]
    tile = tiles[seed % len(tiles)]
    monkeypatch.setenv("ETIR_TILE", str(tile))
    if tile in (7, 8):
        monkeypatch.setenv("ETIR_DMA_VARIANT", str(seed % 2))
    print(f"random forced tile {seed}: {expr} {sizes} dtype {dtype}/{dtype_out} touch {first}/{last} "
          f"tile {tile}", flush=True)
    _, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=dtype, first=first, last=last, seed=seed,
                       dtype_out=dtype_out)
    print(f"  ran: {desc}", flush=True)


@pytest.mark.parametrize("seed", range(6))
def test_random_binary_large(torch_cuda, oracle, seed):
    """Random layouts with at least 256 output tiles of 256 x 256 (the size at
    which the planner chooses its largest tiles) and a short K."""
    rng = np.random.default_rng(4000 + seed)
    letters = list(string.ascii_lowercase)
    rng.shuffle(letters)
    c, m, n, k = letters[0:1], letters[1:3], letters[3:5], letters[5:6 + seed % 2]
    sizes = {c[0]: int(rng.choice([1, 2, 4]))}
    mn = (1 << 24) // sizes[c[0]]
    m0 = int(rng.choice([16, 32, 64, 128, 256]))
    sizes.update({m[0]: m0, m[1]: int(np.sqrt(mn)) // m0})
    n0 = int(rng.choice([16, 32, 64, 128, 256]))
    sizes.update({n[0]: n0, n[1]: int(np.sqrt(mn)) // n0})
    for d in k:
        sizes[d] = int(rng.choice([4, 8, 16, 24])) if len(k) == 1 else int(rng.choice([2, 4, 6]))
    left = list(rng.permutation(c + m + k))
    right = list(rng.permutation(c + n + k))
    out = list(rng.permutation(c + m + n))
    expr = "".join(left) + "," + "".join(right) + "->" + "".join(out)
    dtype = [eir.BF16, eir.FP32][seed % 2]
    print(f"random large {seed}: {expr} {sizes} dtype {dtype}", flush=True)
    _, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=dtype, seed=seed)
    print(f"  ran: {desc}", flush=True)


@pytest.mark.parametrize("seed", range(100))
def test_random_permute(torch_cuda, oracle, seed):
    rng = np.random.default_rng(2000 + seed)
    rank = int(rng.integers(1, 7))
    dims = list(string.ascii_lowercase[:rank])
    sizes = _draw_sizes(rng, dims, 1 << 21)
    out = "".join(rng.permutation(dims))
    dtype = [eir.FP32, eir.FP64, eir.BF16][seed % 3]
    print(f"random permute {seed}: {''.join(dims)}->{out} {sizes} dtype {dtype}", flush=True)
    ktype = eir.ADD if seed % 5 == 4 and dtype != eir.BF16 else eir.COPY
    permute_check(torch_cuda, oracle, "".join(dims) + "->" + out, sizes, dtype=dtype, ktype=ktype, seed=seed)


def _path_cost(ins, sizes, path):
    live = [set(t) for t in ins]
    cost = 0
    for i, j in path:
        u = live[i] | live[j]
        cost += int(np.prod([sizes[d] for d in u]))
        live = [t for k, t in enumerate(live) if k not in (i, j)] + [u]
    return cost


def _tree_case(seed):
    """A random tensor network: every dim sits in two inputs, or in one input
    and the output, or (hyperedges) in three inputs; a random pairwise path."""
    rng = np.random.default_rng(3000 + seed)
    n_in = int(rng.integers(2, 6))
    n_dims = int(rng.integers(n_in + 1, n_in + 6))
    dims = list(string.ascii_lowercase[:n_dims])
    ins = [[] for _ in range(n_in)]
    out = []
    for d in dims:
        r = rng.random()
        if r < 0.3:
            ins[int(rng.integers(0, n_in))].append(d)
            out.append(d)
        elif r < 0.4 and n_in >= 3:
            for a in rng.choice(n_in, 3, replace=False):
                ins[a].append(d)
            if rng.random() < 0.5:
                out.append(d)
        else:
            for a in rng.choice(n_in, 2, replace=False):
                ins[a].append(d)
    extra = iter(string.ascii_uppercase)
    for i, t in enumerate(ins):
        if not t:                       # an empty input shares a new dim with its neighbour
            d = next(extra)
            t.append(d)
            ins[(i + 1) % n_in].append(d)
    if not out:                         # no scalar outputs: give the output a dim of input 0
        d = next(extra)
        ins[0].append(d)
        out.append(d)
    all_dims = sorted(set(d for t in ins for d in t))
    sizes = {d: int(rng.choice([1, 2, 3, 4, 5, 8, 16])) for d in all_dims}
    path, live = [], n_in
    while live > 1:
        i, j = sorted(rng.choice(live, 2, replace=False))
        path.append((int(i), int(j)))
        live -= 1
    ins_s = ["".join(rng.permutation(t)) for t in ins]
    _shrink(sizes, lambda s: _path_cost(ins_s, s, path) + sum(tensor_numel(t, s) for t in ins_s), 1 << 22)
    return ",".join(ins_s) + "->" + "".join(rng.permutation(out)), sizes, path


@pytest.mark.parametrize("seed", range(60))
def test_random_tree(torch_cuda, oracle, seed):
    """fp32 trees against the fp64 path oracle; every third seed a bf16 tree
    (bf16 inputs, intermediates and output, fp32 accumulation) against the
    path oracle that rounds every step's result to bf16 on the same inputs."""
    torch = torch_cuda
    expr, sizes, path = _tree_case(seed)
    bf16 = seed % 3 == 2
    ins, out = expr.split("->")
    print(f"random tree {seed}: {expr} {sizes} {path} {'bf16' if bf16 else 'fp32'}", flush=True)
    rng = np.random.default_rng(seed)
    arrays = [rng.uniform(-1, 1, tensor_numel(t, sizes)).astype(np.float32) for t in ins.split(",")]
    if bf16:
        bits = [oracle.f32_to_bf16(a) for a in arrays]
        dev = [torch.from_numpy(b.view(np.int16)).cuda() for b in bits]
        dout = torch.zeros(tensor_numel(out, sizes), dtype=torch.int16, device="cuda")
        arrays = [oracle.bf16_to_f32(b) for b in bits]
    else:
        dev = [torch.from_numpy(a).cuda() for a in arrays]
        dout = torch.zeros(tensor_numel(out, sizes), dtype=torch.float32, device="cuda")
    e = host.Expression(expr, sizes, path, dev + [dout], dtype=eir.BF16 if bf16 else eir.FP32)
    e.eval()
    got = dout.cpu().numpy()
    if bf16:
        got = oracle.bf16_to_f32(got.view(np.uint16))
    ref = oracle.contract_path(expr, sizes, path, arrays, round_bf16=bf16)
    tol = TOL_BF16 if bf16 else TOL_FP32
    assert rel_frobenius(ref, got) <= tol, f"{expr} {sizes} {path}"
    e.close()
