"""The C++ harness gat_bench (modes and output lines of baseline/bench/main.cpp)."""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from make_smoke1024 import smoke1024, smoke1024_bytes

ROOT = Path(__file__).resolve().parent.parent
BENCH = ROOT / "gat-tfs_amd" / "lib" / "gat_bench"


def run(*args, check_rc=None):
    p = subprocess.run([str(BENCH), *map(str, args)], capture_output=True, text=True, timeout=300)
    if check_rc is not None:
        assert p.returncode == check_rc, (p.returncode, p.stdout[-2000:], p.stderr[-2000:])
    return p


@pytest.fixture(scope="module")
def smoke_file(tmp_path_factory):
    d = tmp_path_factory.mktemp("smoke")
    f = d / "smoke1024.gatbin"
    f.write_bytes(smoke1024_bytes())
    return f


def test_inspect_reads_gatbin(smoke_file):
    p = run("--mode", "inspect", "--graph", smoke_file, "--seed", 11, check_rc=0)
    assert "STATIC N=1024 E=41540 D=128 C=40" in p.stdout


def test_saved_weights_equal_oracle_random_model(smoke_file, tmp_path):
    """Both restate random_model (common.cpp:50-62); the GATWGT1 bytes match."""
    run("--mode", "inspect", "--graph", smoke_file, "--seed", 11, "--save-weights", tmp_path / "h.bin", check_rc=0)
    oracle.save_model(tmp_path / "o.bin", oracle.random_model(128, 40, 11))
    assert (tmp_path / "h.bin").read_bytes() == (tmp_path / "o.bin").read_bytes()
    p = run("--mode", "inspect", "--graph", smoke_file, "--weights", tmp_path / "h.bin", check_rc=0)
    assert "checkpoint=" + str(tmp_path / "h.bin") in p.stdout


def test_saved_graph_roundtrip(tmp_path):
    run("--mode", "inspect", "--synthetic", "uniform:500:8:3", "--din", 16, "--classes", 5, "--seed", 1,
        "--save-graph", tmp_path / "g.gatbin", check_rc=0)
    g = oracle.load_graph(tmp_path / "g.gatbin")
    assert g["n"] == 500 and g["din"] == 16 and g["classes"] == 5 and g["row"][-1] == g["e"]


@pytest.mark.parametrize("defect", ["nonmonotone", "source_oob", "nan_feature", "bad_magic", "truncated"])
def test_malformed_graph_rejected(tmp_path, defect):
    """Graph::validate negative cases (baseline/tests/boundaries.cpp:55-57)."""
    g = smoke1024()
    row, col, x = g["row"].copy(), g["col"].copy(), g["x"].copy()
    if defect == "nonmonotone":
        row[3] = row[-1] + 1
    elif defect == "source_oob":
        col[0] = g["n"]
    elif defect == "nan_feature":
        x[0, 0] = np.nan
    f = tmp_path / "bad.gatbin"
    oracle.save_graph(f, row, col, x, g["classes"])
    if defect == "bad_magic":
        b = bytearray(f.read_bytes())
        b[0:7] = b"XXXXXXX"
        f.write_bytes(bytes(b))
    elif defect == "truncated":
        f.write_bytes(f.read_bytes()[:-100])
    p = run("--mode", "inspect", "--graph", f, "--seed", 11)
    assert p.returncode == 1 and p.stderr.startswith("FAIL")


@pytest.mark.parametrize("argv,msg", [
    (["--mode", "inspect", "--mode", "inspect"], "duplicate argument"),
    (["--bogus", "1"], "unknown option"),
    (["--path", "cpu_fp32", "--graph", "x"], "bad path"),
    (["--mode", "bench"], "bad mode"),
    (["--mode"], "arguments must be --key value"),
])
def test_argument_errors(argv, msg):
    p = run(*argv)
    assert p.returncode == 1 and msg in p.stderr


def test_wrong_checkpoint_shape(smoke_file, tmp_path):
    m = oracle.random_model(64, 40, 11)  # layer 0 in=64, graph din=128
    oracle.save_model(tmp_path / "w.bin", m)
    p = run("--mode", "inspect", "--graph", smoke_file, "--weights", tmp_path / "w.bin")
    assert p.returncode == 1 and "checkpoint model shape mismatch" in p.stderr


def write_r0_dumps(prefix, g, model):
    """R0 stage dumps in the reference's --dump-prefix naming
    (<prefix>_layer<l>_<stage>.f32, baseline/bench/main.cpp:74-77)."""
    x = g["x"]
    for l, p in enumerate(model):
        r = oracle.ref_layer(g["row"], g["col"], x, p, l < 2, edge_stages=True)
        for stage, key in (("output", "out"), ("z", "z"), ("left", "left"), ("right", "right"), ("max", "max"),
                           ("den", "den"), ("p", "p")):
            r[key].astype("<f4").tofile(f"{prefix}_layer{l + 1}_{stage}.f32")
        x = r["out"]


@pytest.mark.gpu
@pytest.mark.parametrize("path,gate", [("gpu_fp32", ("1e-4", "1e-4")), ("gpu_bf16", ("5e-2", "1e-2"))])
def test_correctness_mode_against_r0_dumps(smoke_file, tmp_path, path, gate):
    g = smoke1024()
    model = oracle.random_model(128, 40, 11)
    write_r0_dumps(tmp_path / "r0", g, model)
    p = run("--mode", "correctness", "--graph", smoke_file, "--seed", 11, "--path", path,
            "--reference-prefix", tmp_path / "r0", "--max-abs", gate[0], "--rel-l2", gate[1], check_rc=0)
    assert "CORRECTNESS finite=1 accuracy_gate=PASS" in p.stdout
    assert p.stdout.count("ERROR path=" + path) >= 3 * 5 + 1


@pytest.mark.gpu
def test_benchmark_and_micro_modes(smoke_file, tmp_path):
    p = run("--mode", "benchmark", "--graph", smoke_file, "--seed", 11, "--repeats", 3, "--warmups", 1,
            "--output", tmp_path / "logits.f32", check_rc=0)
    assert "SUMMARY path=gpu_bf16 median_ms=" in p.stdout and p.stdout.count("E2E path=") == 3
    assert p.stdout.count("COLD startup_before_inference_ms=") == 1
    # per-layer JSON of every timed repeat (baseline/bench/main.cpp:177)
    recs = [json.loads(line) for line in p.stdout.splitlines() if line.startswith("{")]
    assert [(r["rep"], r["layer"]) for r in recs] == [(r, l) for r in range(3) for l in (1, 2, 3)]
    assert all(r["mode"] == "benchmark" and r["total_ms"] > 0 and r["score_exp_aggregate_ms"] > 0 for r in recs)
    assert all(r["N"] == 1024 and r["E"] == 41540 for r in recs)
    logits = np.fromfile(tmp_path / "logits.f32", np.float32)
    assert logits.size == 1024 * 40 and np.isfinite(logits).all()
    p = run("--mode", "micro", "--graph", smoke_file, "--seed", 11, "--repeats", 2, "--warmups", 1,
            "--path", "gpu_fp32", check_rc=0)
    assert "MICRO name=prescan_softmax_aggregate_finish layer=2" in p.stdout


@pytest.mark.gpu
def test_export_fixture_roundtrip(smoke_file, tmp_path):
    g = smoke1024()
    model = oracle.random_model(128, 40, 11)
    write_r0_dumps(tmp_path / "r0", g, model)
    run("--mode", "export-fixture", "--graph", smoke_file, "--seed", 11, "--layer", 2,
        "--reference-prefix", tmp_path / "r0", "--fixture", tmp_path / "l2.fix", check_rc=0)
    b = (tmp_path / "l2.fix").read_bytes()
    assert b[:7] == b"GATFIX1"


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["gpu_fp32", "gpu_bf16"])
def test_fixed_p_mode(smoke_file, tmp_path, path):
    """export-fixture then fixed-p (baseline/bench/main.cpp:103-150): the GPU
    standard operator against the FP32 fixed-p master computed by the oracle."""
    g = smoke1024()
    model = oracle.random_model(128, 40, 11)
    write_r0_dumps(tmp_path / "r0", g, model)
    run("--mode", "export-fixture", "--graph", smoke_file, "--seed", 11, "--layer", 2,
        "--reference-prefix", tmp_path / "r0", "--fixture", tmp_path / "l2.fix", check_rc=0)
    x1 = np.fromfile(f"{tmp_path / 'r0'}_layer1_output.f32", np.float32).reshape(1024, -1)
    P = np.fromfile(f"{tmp_path / 'r0'}_layer2_p.f32", np.float32).reshape(-1, 8)
    den = np.fromfile(f"{tmp_path / 'r0'}_layer2_den.f32", np.float32).reshape(1024, 8)
    master = oracle.fixed_p_layer(g["row"], g["col"], x1, model[1], P, den, False)["out"]
    master.astype("<f4").tofile(tmp_path / "master.f32")
    p = run("--mode", "fixed-p", "--graph", smoke_file, "--seed", 11, "--layer", 2, "--path", path,
            "--fixture", tmp_path / "l2.fix", "--reference", tmp_path / "master.f32", "--repeats", 3,
            "--warmups", 1, check_rc=0)
    line = next(l for l in p.stdout.splitlines() if "stage=vs_master_fixed_p" in l)
    fields = dict(kv.split("=") for kv in line.split()[1:])
    if path == "gpu_fp32":
        assert float(fields["max_abs"]) < 1e-4, line
    else:
        assert float(fields["relative_l2"]) < 1e-2, line
    assert f"FIXED_P path={path} layer=2 median_ms=" in p.stdout
    if path == "gpu_bf16":  # layer 2 is 256 -> 8x32: in > 128, so no tfs_op
        assert "median_tfs_ms" not in p.stdout


@pytest.mark.gpu
def test_fixed_p_mode_runs_tfs_operator_on_layer1(smoke_file, tmp_path):
    """Layer 1 of the smoke model (128 -> 8x32) takes both operators of the
    reference's fixed-p mode: standard_op and the neighbour-step tfs_op."""
    g = smoke1024()
    model = oracle.random_model(128, 40, 11)
    write_r0_dumps(tmp_path / "r0", g, model)
    run("--mode", "export-fixture", "--graph", smoke_file, "--seed", 11, "--layer", 1,
        "--reference-prefix", tmp_path / "r0", "--fixture", tmp_path / "l1.fix", check_rc=0)
    P = np.fromfile(f"{tmp_path / 'r0'}_layer1_p.f32", np.float32).reshape(-1, 8)
    den = np.fromfile(f"{tmp_path / 'r0'}_layer1_den.f32", np.float32).reshape(1024, 8)
    master = oracle.fixed_p_layer(g["row"], g["col"], g["x"], model[0], P, den, False)["out"]
    master.astype("<f4").tofile(tmp_path / "master.f32")
    p = run("--mode", "fixed-p", "--graph", smoke_file, "--seed", 11, "--layer", 1, "--path", "gpu_bf16",
            "--fixture", tmp_path / "l1.fix", "--reference", tmp_path / "master.f32", "--repeats", 2,
            "--warmups", 1, check_rc=0)
    lines = {l.split()[1] + " " + l.split()[3]: dict(kv.split("=") for kv in l.split()[1:])
             for l in p.stdout.splitlines() if l.startswith("ERROR")}
    for key in ("path=gpu_bf16_fixed_p stage=vs_master_fixed_p", "path=tfs_b1_fixed_p stage=vs_master_fixed_p"):
        assert float(lines[key]["relative_l2"]) < 1e-2, (key, lines[key])
    assert "median_tfs_ms=" in p.stdout and "speedup=" in p.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("path,precision", [("gpu_fp32", 0), ("gpu_bf16", 1)])
def test_dump_prefix_writes_path_stages(smoke_file, tmp_path, path, precision):
    """--dump-prefix in correctness mode: the path's stages per layer
    (<prefix>_<path>_layer<l>_<stage>.f32) and its chained logits
    (<prefix>_model_<path>.f32, the reference's name, main.cpp:96), equal bit
    for bit to what the C ABI returns for the same layer inputs (the R0-chained
    inputs of correctness mode, main.cpp:71-90)."""
    import gatgpu

    g = smoke1024()
    model = oracle.random_model(128, 40, 11)
    write_r0_dumps(tmp_path / "r0", g, model)
    run("--mode", "correctness", "--graph", smoke_file, "--seed", 11, "--path", path,
        "--reference-prefix", tmp_path / "r0", "--dump-prefix", tmp_path / "d", check_rc=0)
    n = g["n"]
    with gatgpu.Context(0) as ctx:
        ctx.set_graph(g["row"], g["col"])
        ctx.set_model(model)
        ctx.set_input(g["x"])
        x = g["x"]
        for l, p in enumerate(model):
            ctx.layer_forward(l, precision, gatgpu.AUTO, l < 2, input=x)
            for stage, key in (("output", "out"), ("z", "z"), ("left", "left"), ("right", "right"), ("max", "max"),
                               ("den", "den")):
                f = tmp_path / f"d_{path}_layer{l + 1}_{stage}.f32"
                want = ctx.stage(l, key)
                if want is None:  # no Z stage in the aggregate-first dataflow
                    assert not f.exists(), f
                    continue
                got = np.fromfile(f, np.float32)
                assert got.size == want.size, (f, got.size, want.size)
                assert np.array_equal(got, want.ravel()), f
            x = np.fromfile(f"{tmp_path / 'r0'}_layer{l + 1}_output.f32", np.float32).reshape(n, -1)
        logits, _, _ = ctx.model_forward(precision, gatgpu.AUTO)
    got = np.fromfile(tmp_path / f"d_model_{path}.f32", np.float32)
    assert got.size == n * 40 and np.array_equal(got, logits.ravel())
