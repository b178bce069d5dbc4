"""Job files and running a matmul_cluster job on one pod.

`parse_job` reads the scheduler's job-file format (phobos-sched/src/job.rs:5-130):

    source = <path to .ph>          the kernel source (read as text)
    dim NAME = <int>
    tensor NAME = <read|write|rmw> <f16|f32|f64|i8|i32|i64|bool> <D0xD1..> <uri>
    scalar NAME = <f32|f64|i32|i64|bool> <value>

with `#` comments, blank lines ignored and the same errors
("<path>:<line>: <message>").  `run_job` runs a job whose kernel is the
matmul_cluster program (examples/matmul_cluster_fp32.ph: dims M, N, K; A read,
B read, C rmw; alpha, beta) on one pod, with the planner's lowering of
`cluster.lower_matmul` and the @cluster supertile sizes given by the caller.

    python -m phobos_amd.job <job-file> [--tiles TMxTNxTK] [--arena-mib N]
"""
import sys

from . import PhxError
from . import cluster

DTYPES = ("f16", "f32", "f64", "i8", "i32", "i64", "bool")
MODES = ("read", "write", "rmw")


class JobError(ValueError):
    pass


def parse_shape(s):
    """phobos_base::shape::parse: `D0xD1..`, extents trimmed."""
    out = []
    for d in s.split("x"):
        try:
            out.append(int(d.strip()))
        except ValueError:
            raise JobError(f"bad shape extent '{d}'") from None
        if out[-1] < 0:
            raise JobError(f"bad shape extent '{d}'")
    return out


def _scalar(dtype, value):
    bad = JobError(f"scalar value '{value}' is not a valid {dtype}")
    try:
        if dtype in ("f32", "f64"):
            return float(value)
        if dtype in ("i32", "i64"):
            v = int(value)
            bits = 32 if dtype == "i32" else 64
            if not -(1 << (bits - 1)) <= v < (1 << (bits - 1)):
                raise bad
            return v
    except ValueError:
        raise bad from None
    if dtype == "bool":
        if value not in ("true", "false"):
            raise bad
        return value == "true"
    raise JobError(f"unknown scalar data type '{dtype}'")


def parse_job(path, read_source=True):
    """Returns {"source", "source_path", "dimensions", "tensors", "scalars"};
    dimensions and scalars are ordered lists of (name, value) / (name, dtype,
    value), tensors a list of dicts (name, mode, data_type, shape, uri)."""
    with open(path) as f:
        text = f.read()
    job = {"source": None, "source_path": None, "dimensions": [], "tensors": [], "scalars": []}
    for lineno, raw in enumerate(text.splitlines(), 1):
        line = raw.split("#", 1)[0].strip()
        if not line:
            continue

        def err(msg):
            return JobError(f"{path}:{lineno}: {msg}")

        if line.startswith("source"):
            rest = line[len("source"):].lstrip()
            if not rest.startswith("="):
                raise err("expected `source = <path>`")
            src = rest[1:].strip()
            job["source_path"] = src
            if read_source:
                try:
                    with open(src) as f:
                        job["source"] = f.read()
                except OSError as e:
                    raise err(f"reading source file '{src}': {e}") from None
            else:
                job["source"] = ""
        elif line.startswith("dim "):
            name, eq, value = line[4:].partition("=")
            if not eq:
                raise err("expected `dim NAME = VALUE`")
            try:
                v = int(value.strip())
            except ValueError:
                raise err("dim value must be an integer") from None
            job["dimensions"].append((name.strip(), v))
        elif line.startswith("tensor "):
            name, eq, spec = line[7:].partition("=")
            if not eq:
                raise err("expected `tensor NAME = MODE DATA_TYPE SHAPE URI`")
            parts = spec.split()
            for i, what in enumerate(("mode", "data type", "shape", "uri")):
                if len(parts) <= i:
                    raise err(f"tensor missing {what}")
            mode, dtype, shape, uri = parts[:4]
            if mode not in MODES:
                raise err(f"unknown tensor mode '{mode}' (read|write|rmw)")
            if dtype not in DTYPES:
                raise err(f"unknown data type '{dtype}'")
            try:
                shp = parse_shape(shape)
            except JobError as e:
                raise err(str(e)) from None
            job["tensors"].append({"name": name.strip(), "mode": mode, "data_type": dtype,
                                   "shape": shp, "uri": uri})
        elif line.startswith("scalar "):
            name, eq, spec = line[7:].partition("=")
            if not eq:
                raise err("expected `scalar NAME = DATA_TYPE VALUE`")
            parts = spec.split()
            if not parts:
                raise err("scalar missing data type")
            if len(parts) < 2:
                raise err("scalar missing value")
            try:
                v = _scalar(parts[0], parts[1])
            except JobError as e:
                raise err(str(e)) from None
            job["scalars"].append((name.strip(), parts[0], v))
        else:
            raise JobError(f"{path}:{lineno}: unknown directive '{line}'")
    if job["source"] is None:
        raise JobError("job-file has no `source =` line")
    return job


def matmul_job_params(job):
    """Checks that the job is the matmul_cluster program's and returns its
    (M, N, K, alpha, beta, {A|B|C: (uri, shape)})."""
    dims = dict(job["dimensions"])
    tens = {t["name"]: t for t in job["tensors"]}
    sc = {n: v for n, _, v in job["scalars"]}
    for d in ("M", "N", "K"):
        if d not in dims:
            raise JobError(f"matmul job needs dim {d}")
    M, N, K = dims["M"], dims["N"], dims["K"]
    want = {"A": ("read", [M, K]), "B": ("read", [K, N]), "C": ("rmw", [M, N])}
    for name, (mode, shape) in want.items():
        t = tens.get(name)
        if t is None:
            raise JobError(f"matmul job needs tensor {name}")
        if t["mode"] != mode or t["data_type"] != "f32" or t["shape"] != shape:
            raise JobError(f"tensor {name} must be `{mode} f32 {'x'.join(map(str, shape))}`, "
                           f"got `{t['mode']} {t['data_type']} {'x'.join(map(str, t['shape']))}`")
    for s in ("alpha", "beta"):
        if s not in sc:
            raise JobError(f"matmul job needs scalar {s}")
    return M, N, K, float(sc["alpha"]), float(sc["beta"]), {
        n: (tens[n]["uri"], want[n][1]) for n in want}


def run_job(job, tiles=(4096, 8192, 4096), arena_bytes=None, nstreams=4):
    """Runs a matmul_cluster job on one pod; returns the pod's stats."""
    M, N, K, alpha, beta, tens = matmul_job_params(job)
    TM, TN, TK = (min(t, d) for t, d in zip(tiles, (M, N, K)))
    if M % TM or N % TN or K % TK:
        raise JobError(f"supertiles {TM}x{TN}x{TK} must divide M={M}, N={N}, K={K}")
    instrs = cluster.lower_matmul(M, N, K, TM, TN, TK, alpha, beta)
    if arena_bytes is None:
        arena_bytes = 4 * (M * K + K * N + M * N) + (1 << 20)
    pod = cluster.Pod(arena_bytes, nstreams)
    try:
        for idx, name in ((cluster.A, "A"), (cluster.B, "B"), (cluster.C, "C")):
            uri, shape = tens[name]
            pod.set_tensor(idx, uri, shape)
        pod.set_kernel(cluster.STEP_LEAF, cluster.MATMUL)
        pod.set_kernel(cluster.INIT_LEAF, cluster.MATMUL_INIT)
        return pod.run(cluster.segment_text(instrs))
    finally:
        pod.close()


def main(argv=None):
    import argparse
    ap = argparse.ArgumentParser(prog="python -m phobos_amd.job")
    ap.add_argument("job")
    ap.add_argument("--tiles", default="4096x8192x4096", help="@cluster TILE_MxTILE_NxTILE_K")
    ap.add_argument("--arena-mib", type=int, default=None)
    a = ap.parse_args(argv)
    try:
        job = parse_job(a.job)
        tiles = parse_shape(a.tiles)
        if len(tiles) != 3:
            raise JobError("--tiles is TMxTNxTK")
        from . import init
        init(0)
        stats = run_job(job, tiles, None if a.arena_mib is None else a.arena_mib << 20)
    except (JobError, PhxError, OSError) as e:
        print(f"error: {e}", file=sys.stderr)
        return 1
    print(" ".join(f"{k}={v}" for k, v in stats.items()))
    return 0


if __name__ == "__main__":
    sys.exit(main())
