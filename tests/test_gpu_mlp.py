"""GPU parity of the reference's bench_mlp tree: a 5-layer MLP built node by
node with EinsumNode (reference src/bench_mlp.cpp:85-307), every hidden layer
a contraction with a bias first touch (COPY of a tensor broadcast over the
batch dims through aux outer sizes of 1) and a ReLU last touch, the output
layer bias only.  Weights are locked into device copies with
store_and_lock_data, as the reference harness does.

The reference loads trained weights from a TorchScript file; there is none
here, so the weights and biases are seeded uniform[-1/sqrt(fan_in),
1/sqrt(fan_in)] (torch.nn.Linear's initialisation) and the input standard
normal, with the reference's shapes (batch 18 x 64 = 1152, features 784 =
8 x 98, hidden 512 = 8 x 64, 10 outputs).  Checker: numpy float64 of
relu(x W^T + b) layer by layer (the reference compares with torch at
rtol 1e-3 / atol 1e-4, bench_mlp.cpp:403-406); bar: relative Frobenius error
<= 1e-5 (fp32).
"""
import numpy as np
import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import host
from tests.helpers import TOL_FP32, rel_frobenius

pytestmark = pytest.mark.gpu

# dim ids and sizes of bench_mlp.cpp:89-121
SIZES = {0: 18, 1: 64, 2: 8, 3: 98, 4: 8, 5: 64, 6: 8, 7: 64, 8: 8, 9: 64, 10: 8, 11: 64, 12: 10}
AUX = {0: 1, 1: 1, 4: 8, 5: 64, 6: 8, 7: 64, 8: 8, 9: 64, 10: 8, 11: 64, 12: 10}
IDS_IN = [0, 1, 2, 3]
IDS_HIDDEN = [[0, 1, 4, 5], [0, 1, 6, 7], [0, 1, 8, 9], [0, 1, 10, 11]]
IDS_OUT = [0, 1, 12]
IDS_W = [[4, 5, 2, 3], [6, 7, 4, 5], [8, 9, 6, 7], [10, 11, 8, 9], [12, 10, 11]]
WIDTHS = [784, 512, 512, 512, 512, 10]
BATCH = 18 * 64


def _params(seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((BATCH, WIDTHS[0])).astype(np.float32)
    ws, bs = [], []
    for fi, fo in zip(WIDTHS[:-1], WIDTHS[1:]):
        lim = 1.0 / np.sqrt(fi)
        ws.append(rng.uniform(-lim, lim, (fo, fi)).astype(np.float32))
        bs.append(rng.uniform(-lim, lim, fo).astype(np.float32))
    return x, ws, bs


def _reference(x, ws, bs):
    h = x.astype(np.float64)
    for layer, (w, b) in enumerate(zip(ws, bs)):
        h = h @ w.astype(np.float64).T + b.astype(np.float64)
        if layer < len(ws) - 1:
            h = np.maximum(h, 0.0)
    return h


def _build(torch, x, ws, bs, out, stream=None):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).cuda()
    t_x, t_w, t_b = dev(x), [dev(w) for w in ws], [dev(b) for b in bs]
    nodes = host.Nodes(SIZES, AUX, stream=stream)
    n_in = nodes.add_leaf(IDS_IN, t_x)
    n_w = [nodes.add_leaf(ids, t) for ids, t in zip(IDS_W, t_w)]
    prev = n_in
    for layer in range(4):
        prev = nodes.add_binary(IDS_HIDDEN[layer], prev, n_w[layer], aux=t_b[layer],
                                first=eir.COPY, main=eir.MADD, last=eir.RELU)
    root = nodes.add_binary(IDS_OUT, prev, n_w[4], tensor=out, aux=t_b[4],
                            first=eir.COPY, main=eir.MADD, last=eir.UNDEFINED_KTYPE)
    nodes.compile(root)
    return nodes, n_w, t_w


def test_mlp_bias_relu_tree(torch_cuda):
    torch = torch_cuda
    x, ws, bs = _params(7)
    out = torch.zeros(BATCH * WIDTHS[-1], dtype=torch.float32, device="cuda")
    nodes, n_w, t_w = _build(torch, x, ws, bs, out)
    for n in n_w:
        nodes.store_and_lock_data(n)
    nodes.eval()
    ref = _reference(x, ws, bs)
    got = out.cpu().numpy().reshape(BATCH, WIDTHS[-1])
    assert rel_frobenius(ref, got) <= TOL_FP32
    # num_ops: 2*B*fo*fi per layer minus nothing (COPY first touch)
    assert nodes.num_ops() == sum(2 * BATCH * fi * fo for fi, fo in zip(WIDTHS[:-1], WIDTHS[1:]))

    # the locked weights are device copies: clobbering the external buffers
    # changes nothing; after unlock the (zeroed) external buffers are read
    for t in t_w:
        t.zero_()
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    nodes.eval()
    assert rel_frobenius(ref, out.cpu().numpy().reshape(BATCH, WIDTHS[-1])) <= TOL_FP32
    for n in n_w:
        nodes.unlock_data(n)
    nodes.eval()
    # zero weights: every hidden layer is relu(bias), the output b4 + W4 relu(..) = b4
    got = out.cpu().numpy().reshape(BATCH, WIDTHS[-1])
    assert np.array_equal(got, np.broadcast_to(bs[4], got.shape))
    nodes.close()


def test_mlp_relu_is_applied(torch_cuda):
    """Biases of -100 drive every hidden unit negative: the ReLU last touch
    zeroes them all, so the output equals its bias exactly."""
    torch = torch_cuda
    x, ws, bs = _params(8)
    bs = [np.full_like(b, -100.0) for b in bs[:-1]] + [bs[-1]]
    out = torch.zeros(BATCH * WIDTHS[-1], dtype=torch.float32, device="cuda")
    nodes, _, _ = _build(torch, x, ws, bs, out)
    nodes.eval()
    got = out.cpu().numpy().reshape(BATCH, WIDTHS[-1])
    assert np.array_equal(got, np.broadcast_to(bs[-1], got.shape))
    nodes.close()


def test_nodes_reject_bad_children(torch_cuda):
    nodes = host.Nodes({0: 4, 1: 4})
    with pytest.raises(eir.EinsumIrError) as err:
        nodes.add_binary([0, 1], 0, 1)
    assert err.value.code == eir.INVALID_ID
    nodes.close()


def test_mlp_graph_replay(torch_cuda):
    """etir_nodes_eval_graph: the tree recorded once and replayed; every
    replay equals eval()'s output bit for bit, with eager evaluations and
    synchronisations between replays; locking and unlocking the weights drops
    the recording, and the next replay follows the new state."""
    torch = torch_cuda
    x, ws, bs = _params(9)
    out = torch.zeros(BATCH * WIDTHS[-1], dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    nodes, n_w, t_w = _build(torch, x, ws, bs, out, stream=s)
    torch.cuda.synchronize()
    nodes.eval()
    ref = out.cpu().numpy()
    assert rel_frobenius(_reference(x, ws, bs), ref.reshape(BATCH, WIDTHS[-1])) <= TOL_FP32
    for r in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        nodes.eval_graph()
        assert np.array_equal(out.cpu().numpy(), ref), f"replay {r} differs from eval()"
        nodes.eval()
        assert np.array_equal(out.cpu().numpy(), ref)
    # locked weights: device copies, so zeroing the external buffers after
    # the lock changes nothing in the new recording's replays
    for n in n_w:
        nodes.store_and_lock_data(n)
    for t in t_w:
        t.zero_()
    torch.cuda.synchronize()
    for r in range(2):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        nodes.eval_graph()
        assert np.array_equal(out.cpu().numpy(), ref), f"locked replay {r} differs"
    # unlocked: the external (zeroed) weights are read again, output = b4
    for n in n_w:
        nodes.unlock_data(n)
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    nodes.eval_graph()
    got = out.cpu().numpy().reshape(BATCH, WIDTHS[-1])
    assert np.array_equal(got, np.broadcast_to(bs[4], got.shape))
    nodes.close()


def test_mlp_graph_needs_a_stream(torch_cuda):
    x, ws, bs = _params(10)
    out = torch_cuda.zeros(BATCH * WIDTHS[-1], dtype=torch_cuda.float32, device="cuda")
    nodes, _, _ = _build(torch_cuda, x, ws, bs, out)
    with pytest.raises(eir.EinsumIrError):
        nodes.eval_graph()
    nodes.close()
