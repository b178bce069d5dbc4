"""CPU checks of the one-pod matmul segment against the planner's rules
(phobos-sched/src/lib.rs:1022-1093) and of the segment text parser."""
import numpy as np
import pytest

from phobos_amd import cluster as cl


def test_plain_matmul_2x2x2_matches_planner_test():
    # lib.rs:1022-1093: 8192^3, 4096 supertiles, C write-only
    ins = cl.lower_matmul(8192, 8192, 8192, 4096, 4096, 4096, 1.0, 0.0, c_rmw=False)
    c = cl.count_ops(ins)
    assert (c["ALLOC"], c["LOAD"], c["COMPUTE"], c["STORE"], c["FREE"]) == (12, 8, 12, 4, 12)
    assert len(ins) == 48
    c00 = cl.tile_id(2, 0, 0)
    chain = [i for i in ins if i["op"] == "COMPUTE" and any(t == c00 for t, _ in i["args"])]
    assert len(chain) == 3
    assert chain[0]["kernel"] == 1 and chain[1]["kernel"] == 0
    assert chain[0]["iid"] in chain[1]["deps"] and chain[1]["iid"] in chain[2]["deps"]
    assert chain[1]["grid"] == (128, 128, 1) and chain[1]["cta"] == (256, 1, 1)
    a01 = cl.tile_id(0, 0, 1)
    free = next(i for i in ins if i["op"] == "FREE" and i["tile"] == a01)
    assert len(free["deps"]) == 2
    store = next(i for i in ins if i["op"] == "STORE" and i["tile"] == c00)
    assert store["deps"] == [chain[2]["iid"]]
    cfree = next(i for i in ins if i["op"] == "FREE" and i["tile"] == c00)
    assert cfree["deps"] == [store["iid"]]


def test_baseline_job_segment_counts():
    # 16384^3, supertiles 4096 / 8192 / 4096, C read-modify-write
    ins = cl.lower_matmul(16384, 16384, 16384, 4096, 8192, 4096, 0.125, 1.5)
    c = cl.count_ops(ins)
    assert (c["ALLOC"], c["LOAD"], c["COMPUTE"], c["STORE"], c["FREE"]) == (32, 32, 40, 8, 32)
    iids = [i["iid"] for i in ins]
    assert iids == list(range(1, len(ins) + 1))
    seen = set()
    for i in ins:
        assert all(d in seen for d in i["deps"])     # validate(): deps precede
        seen.add(i["iid"])
    comp = [i for i in ins if i["op"] == "COMPUTE"]
    assert comp[0]["kernel"] == 1 and comp[0]["scalars"] == [(1, 1.5)]
    assert comp[1]["scalars"] == [(3, 0.125), (4, 1.5)]
    assert comp[1]["grid"] == (128, 256, 1)


def test_segment_text_roundtrip_fields():
    ins = cl.lower_matmul(512, 512, 512, 256, 256, 256, 0.125, 1.5)
    txt = cl.segment_text(ins)
    lines = txt.strip().splitlines()
    assert len(lines) == len(ins)
    first = lines[0].split()
    assert first[2] == "ALLOC" and first[4] == "256x256"
    comp = next(l for l in lines if " COMPUTE " in l).split()
    assert comp[5] == "1:f32:0x3fc00000"           # beta = 1.5
    step = [l for l in lines if " COMPUTE 0 " in l][0].split()
    assert step[5] == "3:f32:0x3e000000,4:f32:0x3fc00000"


def test_tensor_files_roundtrip(tmp_path):
    p = str(tmp_path / "t.tensor")
    cl.init_tensor(p, (64, 96), "random", 5)
    import oracle
    full = np.fromfile(p, np.float32).reshape(64, 96)
    assert np.array_equal(full.ravel(), oracle.lcg_f32(5, 64 * 96))
    reg = cl.read_region(p, (64, 96), (16, 32), (8, 48))
    assert np.array_equal(reg, full[16:24, 32:80])
