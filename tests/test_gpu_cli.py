"""The modules' command-line demos (the reference's CLIs: fast_article_attention.py:761-894,
triton_article_attention.py:640-856, streaming_taylor_coreset_attention.py:762-805) run on the GPU and
print the reference's table columns / lines."""

import pytest

import fast_article_attention as faa
import streaming_taylor_coreset_attention as stc
import triton_article_attention as taa

pytestmark = pytest.mark.gpu


def _table(text):
    lines = [ln for ln in text.strip().splitlines() if " | " in ln]
    header = lines[0].split(" | ")
    return header, [dict(zip(header, ln.split(" | "))) for ln in lines[2:]]


def test_triton_cli_table(capsys):
    taa._demo(taa._parse_args(["--sweep-n", "128", "300", "--repeats", "1", "--compress-stride", "1"]))
    header, rows = _table(capsys.readouterr().out)
    assert header == ["n", "rel_l2_article", "max_abs_article", "rel_l2_flash", "torch_classical_ms",
                      "triton_flash_ms", "triton_article_ms", "coreset_items", "coreset_bytes", "kv_bytes",
                      "score_matrix"]
    assert [r["n"] for r in rows] == ["128", "300"]
    for r in rows:
        # stride 1: the article path is exact up to fp16 inputs (test_triton_article_attention.py:69)
        assert float(r["rel_l2_article"]) < 2e-2 and float(r["rel_l2_flash"]) < 2e-2
        assert float(r["triton_flash_ms"]) > 0 and float(r["triton_article_ms"]) > 0


def test_fast_cli_table(capsys):
    faa._demo(faa._parser().parse_args(["--sweep-n", "256", "--repeats", "1", "--compressor", "none"]))
    header, rows = _table(capsys.readouterr().out)
    assert header[:5] == ["n", "rel_l2", "max_abs", "classical_ms", "fast_ms"]
    assert rows[0]["n"] == "256" and float(rows[0]["rel_l2"]) < 1e-4  # compressor none is exact


def test_streaming_cli_lines(capsys):
    stc._demo(stc._parser().parse_args(["--n", "200", "--block-size", "32"]))
    out = dict(ln.split("=", 1) for ln in capsys.readouterr().out.strip().splitlines())
    assert set(out) == {"relative_l2", "max_abs", "final_state_bytes"}
    assert float(out["relative_l2"]) < 0.1
    assert int(out["final_state_bytes"].replace(",", "")) > 0
