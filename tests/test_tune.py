"""Kernel-variant selection (qlin_tune*): the table and its file on the CPU, the timed
search on the GPU (every variant must give the same output, and runs after tuning are
unchanged)."""
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from open_rknpu2_lm_infer_amd._lib import QLIN_ERR_PARAM, QlinError


def test_table_file_round_trip(tmp_path):
    ql.tune_clear()
    f = tmp_path / "t.txt"
    f.write_text("# comment\n4 2560 19456 1 0 1 8\n8 4096 2560 512 2 0 3\n4 9728 2560 8 1 0 16\n")
    assert ql.tune_load(str(f)) == 3
    assert ql.tune_count() == 3
    g = tmp_path / "u.txt"
    ql.tune_save(str(g))
    ql.tune_clear()
    assert ql.tune_count() == 0
    assert ql.tune_load(str(g)) == 3
    rows = sorted(l for l in g.read_text().splitlines() if not l.startswith("#"))
    assert rows == sorted(["4 2560 19456 1 0 1 8", "8 4096 2560 512 2 0 3", "4 9728 2560 8 1 0 16"])
    ql.tune_clear()


@pytest.mark.parametrize("line", ["4 2560 19456 1 0 1 5", "3 1 1 1 0 0 4", "4 2560 19456 1 3 0 4", "garbage"])
def test_table_file_rejects(tmp_path, line):
    ql.tune_clear()
    f = tmp_path / "bad.txt"
    f.write_text(line + "\n")
    with pytest.raises(QlinError) as e:
        ql.tune_load(str(f))
    assert e.value.rc == QLIN_ERR_PARAM
    with pytest.raises(QlinError):
        ql.tune_load(str(tmp_path / "missing.txt"))
    ql.tune_clear()


@pytest.mark.gpu
def test_tune_search_keeps_outputs(tmp_path):
    """The search runs every variant of the fused decode GEMV, the GEMV from quantized rows
    and the GEMM, checks them against each other inside the library, and the runs after it
    reproduce the untuned outputs."""
    ql.tune_clear()
    ws = ql.Workspace(512, 9728, 19456)
    cases = [(4, 2560, 19456, 1, ql.QLIN_SWIGLU), (8, 4096, 2560, 8, 0), (4, 9728, 2560, 512, 0),
             (8, 2560, 6144, 300, 0)]
    for i, (bits, K, N, M, fl) in enumerate(cases):
        packed, _, sc = synth.make_linear(N, K, bits, 970 + i, device="cuda:0")
        w = ql.Weights.from_packed_device(bits, K, N, packed, sc)
        A = synth.activations(M, K, seed=980 + i, device="cuda:0")
        before = ql.run(ws, w, A, flags=fl)
        ql.tune(ws, w, M, flags=fl, reps=3)
        after = ql.run(ws, w, A, flags=fl)
        torch.cuda.synchronize()
        assert torch.equal(before, after), f"case {i}"
        w.close()
    assert ql.tune_count() == len(cases)
    ql.tune_save(str(tmp_path / "t.txt"))
    ql.tune_clear()
    assert ql.tune_load(str(tmp_path / "t.txt")) == len(cases)
    ql.tune_clear()
    ws.close()
