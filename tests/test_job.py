"""Job files (phobos-sched/src/job.rs) and the phobos-tensor tool
(phobos-cluster/src/bin/phobos-tensor.rs), on the CPU."""
import numpy as np
import pytest

import oracle
from phobos_amd import job as jb
from phobos_amd import tensor as tn

MATMUL_JOB = """\
# a matmul_cluster job
source = {src}
dim M = 512
dim N = 1024    # trailing comment
dim K = 256

tensor A = read  f32 512x256 file://{d}/a.tensor
tensor B = read  f32 256x1024 file://{d}/b.tensor
tensor C = rmw   f32 512x1024 file://{d}/c.tensor
scalar alpha = f32 0.125
scalar beta = f32 1.5
"""


def _write(tmp_path, text, name="job.txt"):
    p = tmp_path / name
    p.write_text(text)
    return str(p)


def test_parse_matmul_job(tmp_path):
    src = tmp_path / "k.ph"
    src.write_text("kernel matmul(...) {}\n")
    j = jb.parse_job(_write(tmp_path, MATMUL_JOB.format(src=src, d=tmp_path)))
    assert j["source"] == "kernel matmul(...) {}\n"
    assert j["dimensions"] == [("M", 512), ("N", 1024), ("K", 256)]
    assert [t["name"] for t in j["tensors"]] == ["A", "B", "C"]
    assert j["tensors"][2] == {"name": "C", "mode": "rmw", "data_type": "f32",
                               "shape": [512, 1024], "uri": f"file://{tmp_path}/c.tensor"}
    assert j["scalars"] == [("alpha", "f32", 0.125), ("beta", "f32", 1.5)]
    M, N, K, alpha, beta, tens = jb.matmul_job_params(j)
    assert (M, N, K, alpha, beta) == (512, 1024, 256, 0.125, 1.5)
    assert tens["B"] == (f"file://{tmp_path}/b.tensor", [256, 1024])


@pytest.mark.parametrize("line,msg", [
    ("frobnicate x", "unknown directive 'frobnicate x'"),
    ("dim M 5", "expected `dim NAME = VALUE`"),
    ("dim M = five", "dim value must be an integer"),
    ("tensor A = read f32", "tensor missing shape"),
    ("tensor A = read f32 4x4", "tensor missing uri"),
    ("tensor A = peek f32 4x4 file://x", "unknown tensor mode 'peek' (read|write|rmw)"),
    ("tensor A = read f8 4x4 file://x", "unknown data type 'f8'"),
    ("tensor A = read f32 4xN file://x", "bad shape extent 'N'"),
    ("scalar a = f32", "scalar missing value"),
    ("scalar a = f32 abc", "scalar value 'abc' is not a valid f32"),
    ("scalar a = i32 3000000000", "scalar value '3000000000' is not a valid i32"),
    ("scalar a = bool yes", "scalar value 'yes' is not a valid bool"),
    ("scalar a = u8 1", "unknown scalar data type 'u8'"),
    ("source : x", "expected `source = <path>`"),
])
def test_job_errors_name_file_and_line(tmp_path, line, msg):
    p = _write(tmp_path, f"# header\n{line}\n")
    with pytest.raises(jb.JobError) as e:
        jb.parse_job(p, read_source=False)
    assert str(e.value) == f"{p}:2: {msg}"


def test_job_needs_source_and_readable_source(tmp_path):
    with pytest.raises(jb.JobError, match="job-file has no `source =` line"):
        jb.parse_job(_write(tmp_path, "dim M = 1\n"))
    with pytest.raises(jb.JobError, match="reading source file"):
        jb.parse_job(_write(tmp_path, f"source = {tmp_path}/missing.ph\n"))


def test_scalar_kinds(tmp_path):
    p = _write(tmp_path, "source = x\nscalar a = f64 1e-3\nscalar b = i64 -9000000000\n"
                         "scalar c = bool true\nscalar d = i32 -7\n")
    j = jb.parse_job(p, read_source=False)
    assert j["scalars"] == [("a", "f64", 1e-3), ("b", "i64", -9000000000), ("c", "bool", True),
                            ("d", "i32", -7)]


def test_matmul_params_reject_other_programs(tmp_path):
    j = jb.parse_job(_write(tmp_path, MATMUL_JOB.format(src="x", d=tmp_path).replace(
        "tensor C = rmw   f32 512x1024", "tensor C = write f32 512x1024")), read_source=False)
    with pytest.raises(jb.JobError, match="tensor C must be `rmw f32 512x1024`"):
        jb.matmul_job_params(j)


def test_tensor_tool_init_and_peek(tmp_path, capsys):
    uri = f"file://{tmp_path}/sub/t.tensor"
    assert tn.main(["init", "--uri", uri, "--shape", "3x1000", "--fill", "random", "--seed", "2"]) == 0
    got = np.fromfile(f"{tmp_path}/sub/t.tensor", np.float32)
    assert np.array_equal(got, oracle.lcg_f32(2, 3000))      # one Lcg stream (rng.rs)
    assert tn.main(["peek", "--uri", uri, "--shape", "3x1000"]) == 0
    out = capsys.readouterr().out.splitlines()
    assert out[-5].strip() == f"[0,0] = {float(got[0])}"
    assert out[-1].strip() == f"[2,999] = {float(got[-1])}"
    # chunked random fill continues the stream across chunk boundaries
    n = (1 << 20) + 77
    tn.init(f"file://{tmp_path}/big.tensor", [n], "random", seed=5)
    assert np.array_equal(np.fromfile(f"{tmp_path}/big.tensor", np.float32), oracle.lcg_f32(5, n))
    tn.init(f"file://{tmp_path}/i.tensor", [5], "iota")
    assert np.array_equal(np.fromfile(f"{tmp_path}/i.tensor", np.float32), np.arange(5, dtype=np.float32))
    assert tn.main(["init", "--uri", "s3://x", "--shape", "4"]) == 1
    assert tn.file_path("file:///C:/data/x.tensor") == "C:/data/x.tensor"   # storage.rs:14-19
