"""bench.py's contract pieces that run without a GPU: the headline kernel's
measured HBM traffic is read from the committed counter summary only when
that summary was measured on the kernel sources built now (a stale summary
gives no figure), and a multi-GPU request exits with a message instead of
measuring."""

import importlib.util
import json
import pathlib
import subprocess
import sys

REPO = pathlib.Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_contract_probe", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_headline_traffic_row_or_stale():
    b = _bench()
    src = (REPO / "bench.py").read_text()
    assert "counter_traffic(*HEADLINE_KERNEL)" in src
    assert b.HEADLINE_KERNEL == ("norm_modulate_stream_kernel<2, false>", "512")
    text = b.COUNTER_SUMMARY.read_text()
    fresh = f"sources sha256: `{b.source_digest()}`" in text
    t, note = b.counter_traffic(*b.HEADLINE_KERNEL)
    if fresh:
        algorithmic = 2 * 6144 * 4096 * 2 + 2 * 4096 * 2
        assert t is not None and algorithmic <= t <= int(algorithmic * 1.01), (t, note)
    else:
        assert t is None and "kernel sources" in note


def test_stale_summary_gives_no_traffic(monkeypatch):
    b = _bench()
    monkeypatch.setattr(b, "source_digest", lambda: "0000000000000000")
    t, note = b.counter_traffic(*b.HEADLINE_KERNEL)
    assert t is None and "0000000000000000" in note


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=REPO)
    assert r.returncode != 0
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]
