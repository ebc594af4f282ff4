"""GPU tests of concurrent tree evaluation: independent subtrees of an einsum
tree run on streams of their own (ETIR_TREE_STREAMS pool streams, 3 by
default, 0 = every node on the tree's stream).

Each node's kernels are the same either way, so the results must be equal bit
for bit to those of the one-stream evaluation; the forked subtrees use arenas
of their own, so a missing wait shows up as a difference.  The networks are
the reference's einsum_benchmark samples (MERA and the synthetic tree at full
size, the language-model networks at reduced mode sizes), also checked against
torch.einsum in float64 along the same path (relative Frobenius <= 1e-5).
Graph recording (eval_graph) takes the one-stream order.
"""
import json
import os

import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import harness, host
from tests.helpers import TOL_FP32

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
with open(os.path.join(ROOT, "tests", "golden", "einsum_samples.json")) as _f:
    SAMPLES = json.load(_f)["einsum_benchmark"]
REDUCE = {16: 8, 11: 5, 7: 5, 128: 16}


def _case(name):
    c = SAMPLES[name]
    sizes = c["sizes"]
    if name.startswith("lm_"):
        sizes = ",".join(str(REDUCE.get(int(x), int(x))) for x in sizes.split(","))
    ins, out = harness._tensors(c["expr"])
    return c["expr"], ins, out, harness._sizes(c["expr"], sizes), harness._parse_path(c["path"])


def _eval(torch, monkeypatch, name, streams, data, evals=1, stream=None):
    """Output of `evals` back-to-back evaluations on `stream`, the inputs
    negated in place on that stream between them (one snapshot per
    evaluation, copied on the stream)."""
    monkeypatch.setenv("ETIR_TREE_STREAMS", str(streams))
    expr, ins, out, sizes, path = _case(name)
    dout = torch.zeros([sizes[d] for d in out], device="cuda", dtype=torch.float32)
    xs = [d.clone() for d in data]
    torch.cuda.synchronize()
    e = host.Expression(expr, sizes, path, xs + [dout], dtype=eir.FP32, stream=stream)
    snaps = []
    with torch.cuda.stream(stream if stream is not None else torch.cuda.default_stream()):
        for i in range(evals):
            e.eval_async()
            snaps.append(dout.clone())
            if i + 1 < evals:
                xs[i % len(xs)].neg_()
    torch.cuda.synchronize()
    e.close()
    return snaps


@pytest.mark.parametrize("name", ["str_nw_mera_open_26", "synthetic", "lm_first_last_brackets_4_16d",
                                  "lm_batch_likelihood_sentence_5_16d_batch128"])
def test_concurrent_subtrees_bit_equal(torch_cuda, monkeypatch, name):
    torch = torch_cuda
    expr, ins, out, sizes, path = _case(name)
    data = harness.scaled_randn(torch, ins, out, sizes, 7, torch.float32)
    s = torch.cuda.Stream()
    one = _eval(torch, monkeypatch, name, 0, data, stream=s)[0]
    conc = _eval(torch, monkeypatch, name, 4, data, stream=s)[0]
    assert torch.equal(one, conc), "concurrent evaluation differs from the one-stream evaluation"
    ref = harness.torch_path_eval(torch, ins, out, sizes, path, [d.double() for d in data])
    err = float(torch.linalg.vector_norm(ref - conc.double()) / torch.linalg.vector_norm(ref))
    assert err <= TOL_FP32, err


@pytest.mark.parametrize("streams", [1, 4])
def test_back_to_back_evaluations(torch_cuda, monkeypatch, streams):
    """Four evaluations enqueued without waiting, an input changed on the
    tree's stream before each: every snapshot equals the one-stream result for
    the inputs of its turn (a forked subtree of one evaluation may not start
    before the input change, nor overwrite its arena while the previous
    evaluation still reads it)."""
    torch = torch_cuda
    name = "str_nw_mera_open_26"
    expr, ins, out, sizes, path = _case(name)
    data = harness.scaled_randn(torch, ins, out, sizes, 8, torch.float32)
    s = torch.cuda.Stream()
    want = _eval(torch, monkeypatch, name, 0, data, evals=4, stream=s)
    got = _eval(torch, monkeypatch, name, streams, data, evals=4, stream=s)
    assert not torch.equal(want[0], want[1])
    for i, (w, g) in enumerate(zip(want, got)):
        assert torch.equal(w, g), f"evaluation {i} differs"


def test_concurrent_subtrees_null_stream(torch_cuda, monkeypatch):
    """The tree on the null stream forks and joins the same way."""
    torch = torch_cuda
    name = "synthetic"
    expr, ins, out, sizes, path = _case(name)
    data = harness.scaled_randn(torch, ins, out, sizes, 9, torch.float32)
    one = _eval(torch, monkeypatch, name, 0, data, evals=2)
    conc = _eval(torch, monkeypatch, name, 4, data, evals=2)
    for w, g in zip(one, conc):
        assert torch.equal(w, g)


def test_graph_recording_one_stream(torch_cuda, monkeypatch):
    """With forked subtrees in the schedule, eval_graph records the tree on
    its one stream (every kernel there, one-stream order, the forked
    subtrees' arenas as scheduled): every replay equals the eager concurrent
    result, with eager evaluations between the replays."""
    torch = torch_cuda
    monkeypatch.setenv("ETIR_TREE_STREAMS", "4")
    name = "str_nw_mera_open_26"
    expr, ins, out, sizes, path = _case(name)
    data = harness.scaled_randn(torch, ins, out, sizes, 10, torch.float32)
    dout = torch.zeros([sizes[d] for d in out], device="cuda", dtype=torch.float32)
    s = torch.cuda.Stream()
    e = host.Expression(expr, sizes, path, data + [dout], dtype=eir.FP32, stream=s)
    e.eval()
    ref = dout.clone()
    for r in range(3):
        dout.fill_(float("nan"))
        torch.cuda.synchronize()
        e.eval_graph()
        assert torch.equal(dout, ref), f"replay {r} differs from eval()"
        e.eval()
        assert torch.equal(dout, ref)
    e.close()
