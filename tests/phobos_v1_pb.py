"""phobos.v1 message classes built with google.protobuf from a restatement of
the reference's schema (phobos-cluster/proto/v1/phobos_v1_isa.proto:1-110 and
the JobManifest part of phobos_v1_scheduler.proto:53-76), so the tests have an
encoder and decoder independent of this build's own.  Test infrastructure."""
from google.protobuf import descriptor_pb2, descriptor_pool, message_factory

F = descriptor_pb2.FieldDescriptorProto
U64, U32, I32, I64, F32, F64, BOOL, STR, ENUM, MSG = (
    F.TYPE_UINT64, F.TYPE_UINT32, F.TYPE_INT32, F.TYPE_INT64, F.TYPE_FLOAT, F.TYPE_DOUBLE,
    F.TYPE_BOOL, F.TYPE_STRING, F.TYPE_ENUM, F.TYPE_MESSAGE)
REP = "rep"

# message -> [(name, number, type, type_name or None, repeated?, oneof index or None)]
SCHEMA = {
    "Region": [("offset", 1, U64, None, REP), ("shape", 2, U64, None, REP)],
    "StorageReference": [("tensor", 1, U32), ("region", 2, MSG, "Region")],
    "Dim3": [("x", 1, U32), ("y", 2, U32), ("z", 3, U32)],
    "ComputeArgument": [("tile", 1, U64), ("mode", 2, ENUM, "AccessMode")],
    "ScalarValue": [("f32", 1, F32, None, None, 0), ("f64", 2, F64, None, None, 0),
                    ("i32", 3, I32, None, None, 0), ("i64", 4, I64, None, None, 0),
                    ("boolean", 5, BOOL, None, None, 0)],
    "ScalarArgument": [("position", 1, U32), ("value", 2, MSG, "ScalarValue")],
    "Allocate": [("tile", 1, U64), ("shape", 2, U64, None, REP), ("data_type", 3, ENUM, "DataType")],
    "Load": [("tile", 1, U64), ("source", 2, MSG, "StorageReference")],
    "Fetch": [("tile", 1, U64), ("from", 2, U32)],
    "Compute": [("kernel", 1, U32), ("arguments", 2, MSG, "ComputeArgument", REP),
                ("grid", 3, MSG, "Dim3"), ("cta", 4, MSG, "Dim3"),
                ("scalars", 5, MSG, "ScalarArgument", REP)],
    "Store": [("tile", 1, U64), ("destination", 2, MSG, "StorageReference")],
    "Free": [("tile", 1, U64), ("expected_serves", 2, U32)],
    "Operation": [("allocate", 1, MSG, "Allocate", None, 0), ("load", 2, MSG, "Load", None, 0),
                  ("fetch", 3, MSG, "Fetch", None, 0), ("compute", 4, MSG, "Compute", None, 0),
                  ("store", 5, MSG, "Store", None, 0), ("free", 6, MSG, "Free", None, 0)],
    "Instruction": [("iid", 1, U64), ("dependencies", 2, U64, None, REP),
                    ("operation", 3, MSG, "Operation")],
    "Segment": [("id", 1, U64), ("instructions", 2, MSG, "Instruction", REP)],
    "TensorEntry": [("index", 1, U32), ("uri", 2, STR), ("data_type", 3, ENUM, "DataType"),
                    ("shape", 4, U64, None, REP), ("mode", 5, ENUM, "AccessMode")],
    "KernelEntry": [("index", 1, U32), ("hash", 2, STR), ("name", 3, STR)],
    "KernelHolder": [("hash", 1, STR), ("node_id", 2, U32)],
    "JobManifest": [("tensors", 1, MSG, "TensorEntry", REP), ("kernels", 2, MSG, "KernelEntry", REP),
                    ("kernel_holders", 3, MSG, "KernelHolder", REP)],
}
ENUMS = {
    "DataType": ["DATA_TYPE_UNSPECIFIED", "DATA_TYPE_F16", "DATA_TYPE_F32", "DATA_TYPE_F64",
                 "DATA_TYPE_I8", "DATA_TYPE_I32", "DATA_TYPE_I64", "DATA_TYPE_BOOL"],
    "AccessMode": ["ACCESS_MODE_UNSPECIFIED", "ACCESS_MODE_READ", "ACCESS_MODE_WRITE",
                   "ACCESS_MODE_RMW"],
}
ONEOF = {"ScalarValue": "value", "Operation": "kind"}


def _build():
    fd = descriptor_pb2.FileDescriptorProto(name="phobos_v1_test.proto", package="phobos.v1",
                                            syntax="proto3")
    for name, values in ENUMS.items():
        e = fd.enum_type.add(name=name)
        for i, v in enumerate(values):
            e.value.add(name=v, number=i)
    for name, fields in SCHEMA.items():
        m = fd.message_type.add(name=name)
        if name in ONEOF:
            m.oneof_decl.add(name=ONEOF[name])
        for spec in fields:
            fname, num, ftype = spec[:3]
            tname = spec[3] if len(spec) > 3 else None
            rep = len(spec) > 4 and spec[4] == REP
            oneof = spec[5] if len(spec) > 5 else None
            f = m.field.add(name=fname, number=num, type=ftype,
                            label=F.LABEL_REPEATED if rep else F.LABEL_OPTIONAL)
            if tname:
                f.type_name = ".phobos.v1." + tname
            if oneof is not None:
                f.oneof_index = oneof
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fd)
    return {n: message_factory.GetMessageClass(pool.FindMessageTypeByName("phobos.v1." + n))
            for n in SCHEMA}


M = _build()


def segment_from_instrs(instrs, segment_id=0):
    """The lowering's instruction dicts as a Segment message."""
    seg = M["Segment"](id=segment_id)
    am = {"r": 1, "w": 2, "rmw": 3}
    for i in instrs:
        ins = seg.instructions.add(iid=i["iid"], dependencies=i["deps"])
        op = ins.operation
        op.SetInParent()
        if i["op"] == "ALLOC":
            op.allocate.SetInParent()
            op.allocate.tile = i["tile"]
            op.allocate.shape.extend(i["shape"])
            op.allocate.data_type = 2
        elif i["op"] in ("LOAD", "STORE"):
            body = op.load if i["op"] == "LOAD" else op.store
            body.SetInParent()
            ref = body.source if i["op"] == "LOAD" else body.destination
            ref.SetInParent()
            ref.region.SetInParent()
            body.tile = i["tile"]
            ref.tensor = i["tensor"]
            ref.region.offset.extend(i["offset"])
            ref.region.shape.extend(i["shape"])
        elif i["op"] == "COMPUTE":
            c = op.compute
            c.SetInParent()
            c.grid.SetInParent()
            c.cta.SetInParent()
            c.kernel = i["kernel"]
            for t, m in i["args"]:
                c.arguments.add(tile=t, mode=am[m])
            c.grid.x, c.grid.y, c.grid.z = i["grid"]
            c.cta.x, c.cta.y, c.cta.z = i["cta"]
            for pos, v in i["scalars"]:
                c.scalars.add(position=pos).value.f32 = v
        else:
            op.free.SetInParent()
            op.free.tile = i["tile"]
            op.free.expected_serves = i.get("serves", 0)
    return seg
