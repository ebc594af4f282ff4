"""CPU checks of the harness command line (usage and argument errors; no GPU)."""
from einsum_ir_amd import harness


def test_usage_without_arguments(capsys):
    assert harness.main([]) == 1
    assert "python -m einsum_ir_amd.harness binary" in capsys.readouterr().err


def test_unknown_command_and_missing_arguments(capsys):
    assert harness.main(["gemm", "a", "b"]) == 1
    assert harness.main(["expression", "ab,bc->ac", "2,3,4"]) == 1   # no contraction path


def test_tree_parser_post_order():
    nodes = harness._parse_tree("[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]")
    assert nodes == [([3, 0], []), ([0, 3], [0]), ([3, 2, 4], []), ([1, 4, 2], []),
                     ([1, 2, 3], [2, 3]), ([0, 1, 2], [1, 4])]


def test_path_and_tensor_parsing():
    assert harness._parse_path("(1,2),(2,3),(0,1),(0,1)") == [(1, 2), (2, 3), (0, 1), (0, 1)]
    assert harness._tensors("[a,b],[b,c]->[a,c]") == ([["a", "b"], ["b", "c"]], ["a", "c"])
    assert harness._tensors("iae,bf->ab") == ([["i", "a", "e"], ["b", "f"]], ["a", "b"])
