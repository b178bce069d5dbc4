"""The scheduler's wire format: phobos.v1.Segment / JobManifest encoding
(phobos_amd.cluster) and the C++ decoder (phx_segment_pb_to_text, the one
phx_pod_run_segment_pb uses), checked against google.protobuf's own encoding
of the reference schema (phobos-cluster/proto/v1/phobos_v1_isa.proto) and the
checks of segment_from_proto (phobos-cluster/src/proto.rs:193-275).  CPU only."""
import struct

import pytest

import phobos_amd as px
from phobos_amd import cluster
from phobos_v1_pb import M, segment_from_instrs


def _err(data):
    with pytest.raises(px.PhxError) as e:
        px.segment_pb_to_text(data)
    return e.value


@pytest.mark.parametrize("dims", [(512, 512, 512, 256, 256, 256),
                                  (16384, 16384, 16384, 4096, 8192, 4096)])
def test_encoder_is_canonical_protobuf(dims):
    ins = cluster.lower_matmul(*dims, 0.125, 1.5)
    ours = cluster.segment_pb(ins, 7)
    ref = segment_from_instrs(ins, 7).SerializeToString()
    assert ours == ref
    back = M["Segment"].FromString(ours)
    assert back.id == 7 and len(back.instructions) == len(ins)
    assert [i.iid for i in back.instructions] == [i["iid"] for i in ins]


@pytest.mark.parametrize("c_rmw", [True, False])
def test_decoder_round_trip_matches_text_form(c_rmw):
    ins = cluster.lower_matmul(1024, 2048, 1024, 512, 1024, 256, 0.125, 1.5, c_rmw=c_rmw)
    data = segment_from_instrs(ins, 3).SerializeToString()
    assert px.segment_pb_to_text(data) == cluster.segment_text(ins)


def _one_compute(**scalars):
    seg = M["Segment"](id=1)
    ins = seg.instructions.add(iid=5)
    c = ins.operation.compute
    c.kernel = 2
    c.arguments.add(tile=0x10000000000003, mode=3)
    c.grid.SetInParent()
    c.grid.x, c.grid.y, c.grid.z = 4, 2, 1
    c.cta.x = 256
    for pos, (kind, v) in scalars.items():
        setattr(c.scalars.add(position=int(pos[1:])).value, kind, v)
    return seg


def test_decoder_scalar_kinds_keep_bits():
    seg = _one_compute(p3=("f32", 0.125), p4=("i32", -7), p5=("i64", -(1 << 40)),
                       p6=("f64", 2.5), p7=("boolean", True))
    txt = px.segment_pb_to_text(seg.SerializeToString())
    f64_bits = struct.unpack("<q", struct.pack("<d", 2.5))[0]
    assert txt.strip() == (f"5 - COMPUTE 2 0x10000000000003:rmw 3:f32:0x3e000000,"
                           f"4:f32:0xfffffff9,5:i64:{-(1 << 40)},6:i64:{f64_bits},7:bool:1 "
                           f"4,2,1 256,0,0")


def test_decoder_accepts_unpacked_and_skips_unknown_fields():
    ins = cluster.lower_matmul(512, 512, 512, 256, 256, 256, 0.125, 1.5)
    data = cluster.segment_pb(ins, 7)
    # the same deps unpacked (one varint per element) and an unknown field 9
    seg = M["Segment"].FromString(data)
    first = seg.instructions[2]  # has a dependency list
    deps = list(first.dependencies)
    body = first.SerializeToString()
    packed = b"\x12" + bytes([len(deps)]) + bytes(deps)
    assert packed in body
    unpacked = b"".join(b"\x10" + bytes([d]) for d in deps) + b"\x48\x2a"
    body2 = body.replace(packed, unpacked)
    enc = lambda b: b"\x12" + cluster._varint(len(b)) + b
    data2 = data.replace(enc(body), enc(body2))
    assert data2 != data
    assert px.segment_pb_to_text(data2) == cluster.segment_text(ins)


def test_decoder_errors_follow_segment_from_proto():
    def one(build):
        seg = M["Segment"](id=1)
        ins = seg.instructions.add(iid=1)
        build(ins.operation)
        return seg.SerializeToString()

    e = _err(one(lambda op: (op.fetch.SetInParent(), setattr(op.fetch, "tile", 4))))
    assert e.code == 1006 and "FETCH" in str(e)

    def no_grid(op):
        op.compute.SetInParent()
        op.compute.cta.x = 256
    assert "Compute.grid missing" in str(_err(one(no_grid)))

    def no_source(op):
        op.load.SetInParent()
        op.load.tile = 9
    assert "Load.source missing" in str(_err(one(no_source)))

    def bad_mode(op):
        c = op.compute
        c.grid.x = c.cta.x = 1
        c.arguments.add(tile=1, mode=0)
    assert "unknown AccessMode" in str(_err(one(bad_mode)))

    def f16_alloc(op):
        op.allocate.shape.extend([4, 4])
        op.allocate.data_type = 1
    assert "only f32" in str(_err(one(f16_alloc)))

    def no_dtype(op):
        op.allocate.shape.extend([4, 4])
    assert "unknown DataType 0" in str(_err(one(no_dtype)))

    seg = M["Segment"](id=1)
    seg.instructions.add(iid=3)
    assert "Instruction.operation missing" in str(_err(seg.SerializeToString()))

    seg = _one_compute(p3=("f32", 1.0))
    seg.instructions[0].operation.compute.scalars[0].ClearField("value")
    assert "ScalarArgument.value missing" in str(_err(seg.SerializeToString()))

    good = cluster.segment_pb(cluster.lower_matmul(512, 512, 512, 256, 256, 256, 0.125, 1.5))
    for cut in (1, 7, len(good) // 2, len(good) - 1):
        assert _err(good[:cut]).code == 1006


def test_manifest_encoder_is_canonical_protobuf():
    tensors = [(0, "file:///tmp/a.tensor", (1024, 512)), (2, "file:///C:/x/c.tensor", (7,))]
    kernels = [(0, "ab" * 32, "matmul"), (1, "cd" * 32, "matmul_init")]
    ours = cluster.manifest_pb(tensors, kernels)
    ref = M["JobManifest"]()
    for idx, uri, shape in tensors:
        ref.tensors.add(index=idx, uri=uri, data_type=2, shape=shape)
    for idx, h, name in kernels:
        ref.kernels.add(index=idx, hash=h, name=name)
    assert ours == ref.SerializeToString()


def test_decoder_survives_corrupt_input():
    # Mutated, truncated, extended and random encodings: the decoder returns
    # a segment or an error for each, and never reads out of bounds (a crash
    # would end the test run).  Seeded, so the cases are the same every run.
    import random
    ins = cluster.lower_matmul(1024, 2048, 1024, 512, 1024, 256, 0.125, 1.5)
    base = segment_from_instrs(ins, 3).SerializeToString()
    rng = random.Random(20261201)
    decoded = refused = 0
    for _ in range(3000):
        d = bytearray(base)
        kind = rng.randrange(4)
        if kind == 0:
            for _ in range(rng.randrange(1, 8)):
                d[rng.randrange(len(d))] = rng.randrange(256)
        elif kind == 1:
            d = d[:rng.randrange(len(d))]
        elif kind == 2:
            d = bytearray(rng.randrange(256) for _ in range(rng.randrange(64)))
        else:
            at = rng.randrange(len(d))
            d[at:at] = bytes(rng.randrange(256) for _ in range(rng.randrange(1, 16)))
        try:
            px.segment_pb_to_text(bytes(d))
            decoded += 1
        except px.PhxError:
            refused += 1
    assert decoded + refused == 3000 and refused > 0
