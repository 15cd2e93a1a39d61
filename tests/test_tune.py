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


def test_table_gemm_kernel_field(tmp_path):
    """GEMM entries carry splits + 100 * kernel: 0 the planner's pick, 1 the 16x16x64 kernel,
    2..5 the 32x32x32 kernel's tile configurations (5 for W4 only)."""
    ql.tune_clear()
    f = tmp_path / "g.txt"
    lines = ["4 9728 2560 4096 2 0 301", "4 2560 19456 512 2 1 501", "8 4096 2560 512 2 0 103",
             "8 2560 6144 512 2 0 402", "4 2560 6144 64 2 0 64"]
    f.write_text("\n".join(lines) + "\n")
    assert ql.tune_load(str(f)) == len(lines)
    g = tmp_path / "h.txt"
    ql.tune_save(str(g))
    assert sorted(l for l in g.read_text().splitlines() if not l.startswith("#")) == sorted(lines)
    ql.tune_clear()


@pytest.mark.parametrize("line", ["4 2560 19456 1 0 1 5", "3 1 1 1 0 0 4", "4 2560 19456 1 3 0 4", "garbage",
                                  "8 2560 19456 512 2 1 501", "4 2560 19456 512 2 1 601", "4 2560 6144 512 2 0 300",
                                  "4 2560 6144 512 2 0 65", "4 2560 6144 512 2 0 0"])
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
             (8, 2560, 6144, 300, 0), (4, 4096, 2560, 24, 0)]
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
    # the GEMM entries name the kernel the search timed fastest (the 32x32x32 tile
    # configurations exist at 128 x 128, 256 x 256 / 256 x 128, 128 x 256 and, W4 only, 256 x 192)
    f = tmp_path / "t.txt"
    ql.tune_save(str(f))
    gemm = [l.split() for l in f.read_text().splitlines() if not l.startswith("#") and l.split()[4] == "2"]
    assert len(gemm) == 2
    for e in gemm:
        v = int(e[6])
        assert 1 <= v % 100 <= 8 and 1 <= v // 100 <= (5 if e[0] == "4" else 4), e
    ql.tune_clear()


@pytest.mark.gpu
def test_tuned_gemm_kernel_is_planned(tmp_path):
    """A table entry's kernel and splits reach the plan (tile shape and waves name the
    kernel), and the output stays bit-identical to the planner's own choice."""
    ql.tune_clear()
    bits, K, N, M = 4, 9728, 2560, 512
    ws = ql.Workspace(M, K, N)
    packed, _, sc = synth.make_linear(N, K, bits, 990, device="cuda:0")
    w = ql.Weights.from_packed_device(bits, K, N, packed, sc)
    A = synth.activations(M, K, seed=991, device="cuda:0")
    base = ql.run(ws, w, A)
    # kernel field -> (tile rows, tile channels, waves per workgroup)
    shape = {1: (128, 128, 8), 2: (128, 128, 4), 3: (256, 256, 8), 4: (128, 256, 8), 5: (256, 192, 12)}
    f = tmp_path / "one.txt"
    for kern, want in shape.items():
        for splits in (1, 3):
            ql.tune_clear()
            f.write_text(f"{bits} {K} {N} {M} 2 0 {splits + 100 * kern}\n")
            assert ql.tune_load(str(f)) == 1
            pl = ql.plan(ws, w, A)
            assert pl["path"] == ql.QLIN_PATH_GEMM and pl["splits"] == splits, (kern, splits, pl)
            assert (pl["tile_m"], pl["tile_n"], pl["waves"]) == want, (kern, pl)
            out = ql.run(ws, w, A)
            torch.cuda.synchronize()
            assert torch.equal(out, base), (kern, splits)
    ql.tune_clear()
    w.close()
    ws.close()
