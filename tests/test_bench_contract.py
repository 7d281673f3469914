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
    assert b.HEADLINE_KERNEL == ("norm_modulate_wave_kernel<8, false>", "1024")
    text = b.COUNTER_SUMMARY.read_text()
    fresh = f"sources sha256: `{b.source_digest()}`" in text
    t, note = b.counter_traffic(*b.HEADLINE_KERNEL)
    if fresh:
        algorithmic = 2 * 6144 * 4096 * 2 + 2 * 4096 * 2
        # counters calibrated on a device copy: within a few percent of the algorithmic bytes
        assert t is not None and 0.98 * algorithmic <= t <= 1.05 * algorithmic, (t, note)
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


def test_counter_summary_calibrates_on_the_copy(tmp_path):
    """summarize_counters scales FETCH_SIZE and WRITE_SIZE by what they read for
    the device copy of the config-1 activation, and writes the sources line that
    counter_traffic checks; the summary it writes is read back by counter_traffic."""
    b = _bench()
    kib = 6144 * 4096 * 2 / 1024
    head = "Kernel_Name,Grid_Size,Workgroup_Size,Counter_Value\n"
    fetch = head + (f"__amd_rocclr_copyBuffer,65536,256,{kib / 2}\n"
                    f'"void ltxk::(anonymous namespace)::norm_modulate_wave_kernel<8, false>(ltxk::Norm)",'
                    f"262144,256,{kib / 2 + 4}\n")
    write = head + (f"__amd_rocclr_copyBuffer,65536,256,{kib}\n"
                    f'"void ltxk::(anonymous namespace)::norm_modulate_wave_kernel<8, false>(ltxk::Norm)",'
                    f"262144,256,{kib}\n")
    (tmp_path / "f.csv").write_text(fetch)
    (tmp_path / "w.csv").write_text(write)
    md = b.summarize_counters(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), "norm_mod")
    assert f"sources sha256: `{b.source_digest()}`" in md
    assert "fetch factor 2.000, write factor 1.000" in md
    (tmp_path / "sum.md").write_text(md)
    b.COUNTER_SUMMARY = tmp_path / "sum.md"
    t, note = b.counter_traffic(*b.HEADLINE_KERNEL)
    assert t == int(round((2 * (kib / 2 + 4) + kib) * 1024 / 1e6, 2) * 1e6), (t, note)


def test_trace_summary_groups_dispatches(tmp_path):
    b = _bench()
    rows = ["Kernel_Name,Grid_Size_X,Workgroup_Size_X,VGPR_Count,Start_Timestamp,End_Timestamp"]
    for i, d in enumerate((17000, 18000, 19000)):
        rows.append(f'"void ltxk::(anonymous namespace)::norm_modulate_stream_kernel<2, false>(ltxk::Norm)",'
                    f"131072,256,64,{i * 100000},{i * 100000 + d}")
    (tmp_path / "t.csv").write_text("\n".join(rows) + "\n")
    md = b.summarize_trace(str(tmp_path / "t.csv"))
    assert "| `norm_modulate_stream_kernel<2, false>` | 512 | 256 | 64 | 3 | 18.00 | 18.00 |" in md


def test_pmc_summary_means_per_dispatch(tmp_path):
    """summarize_pmc sums a counter's rows of one dispatch (one per XCD or
    instance) before averaging over dispatches, keeps kernels apart by name
    and workgroup count, and forms the two memory-pipeline ratios."""
    b = _bench()
    head = "Dispatch_Id,Kernel_Name,Grid_Size,Workgroup_Size,Counter_Name,Counter_Value\n"
    k = '"void ltxk::(anonymous namespace)::qk_pair_wave_kernel<4>(ltxk::QKParams)"'
    rows = []
    for d, (lvl, act) in enumerate(((300.0, 10.0), (500.0, 10.0))):  # two dispatches, two rows each for LEVEL
        rows += [f"{d},{k},262144,256,TCC_EA0_RDREQ_LEVEL,{lvl}", f"{d},{k},262144,256,TCC_EA0_RDREQ_LEVEL,{lvl}",
                 f"{d},{k},262144,256,GRBM_GUI_ACTIVE,{act}"]
    rows.append("9,flat_kernel<0>,1024,256,GRBM_GUI_ACTIVE,5")
    (tmp_path / "a.csv").write_text(head + "\n".join(rows) + "\n")
    md = b.summarize_pmc([str(tmp_path / "a.csv")], "qk_")
    assert "| TCC_EA0_RDREQ_LEVEL | 800 |" in md       # (600 + 1000) / 2
    assert "| GRBM_GUI_ACTIVE | 10 |" in md
    assert "| reads outstanding (RDREQ_LEVEL / GUI_ACTIVE) | 80 |" in md
    assert "flat_kernel" not in md and "`qk_pair_wave_kernel<4>` 2" in md


def test_buffer_rotation_spans_past_the_mall():
    """Every kernel line rotates enough input/output sets that together they
    span >= 1 GB (4x the 256 MB MALL), so no call reads its operands from
    the MALL: the set count for a few per-set sizes of the bench's lines."""
    b = _bench()
    assert b.ROTATE_BYTES >= 4 * 256 * 2**20
    for per_set in (100_663_296, 50_331_648, 25_690_112, 251_658_240, 805_306_368):
        n = b.nsets(per_set)
        assert n >= 2 and n * per_set >= b.ROTATE_BYTES and (n - 1) * per_set < b.ROTATE_BYTES or n == 2
    assert b.nsets(100_663_296) == 11 and b.nsets(50_331_648) == 22


def test_counter_collection_needs_plain_mode():
    """Under rocprofv3 counter collection (ROCPROF_COUNTER_COLLECTION in the
    environment) bench.py refuses to run without --plain, before touching a GPU."""
    import os

    env = dict(os.environ, ROCPROF_COUNTER_COLLECTION="1")
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--only", "norm_modulate"], capture_output=True,
                       text=True, timeout=120, cwd=REPO, env=env)
    assert r.returncode == 2
    assert "--plain" in json.loads(r.stdout.strip().splitlines()[-1])["error"]
