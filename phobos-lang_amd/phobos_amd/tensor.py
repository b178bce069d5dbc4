"""phobos-tensor: create and inspect the raw f32 tensor files a job reads
(phobos-cluster/src/bin/phobos-tensor.rs:1-130).

    python -m phobos_amd.tensor init --uri <file://...> --shape <RxC|N>
                                     [--fill zero|random|const|iota] [--value f] [--seed s]
    python -m phobos_amd.tensor peek --uri <file://...> --shape <RxC|N>

Files are row-major little-endian f32; `random` is the Lcg stream of the
example harnesses (uniform [-1, 1), seed default 1), written in 1 Mi-element
chunks so a 1 GiB tensor never sits in memory whole.  `peek` prints the
corners and the centre."""
import os
import sys

import numpy as np

from .job import JobError, parse_shape

USAGE = __doc__.split("\n\n")[1]
CHUNK = 1 << 20


def file_path(uri):
    """storage::file_path: file:// only; "/C:..." drops its leading '/'."""
    if not uri.startswith("file://"):
        raise JobError(f"unsupported storage URI '{uri}' (expected file://)")
    rest = uri[len("file://"):]
    if rest.startswith("/") and len(rest) > 2 and rest[2] == ":":
        rest = rest[1:]
    return rest


def init(uri, shape, fill="zero", value=0.0, seed=1):
    from . import lib, check
    import ctypes
    if fill not in ("zero", "random", "const", "iota"):
        raise JobError(f"unknown --fill '{fill}'")
    total = int(np.prod(shape)) if shape else 0
    path = file_path(uri)
    if os.path.dirname(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "wb") as f:
        if fill == "random":
            # one Lcg stream over the whole tensor: draw it chunk by chunk
            state = ctypes.c_uint64(seed)
            buf = np.empty(min(CHUNK, max(total, 1)), np.float32)
            done = 0
            while done < total:
                n = min(CHUNK, total - done)
                check(lib().phx_lcg_fill_f32_stream(ctypes.byref(state), n,
                                                     buf.ctypes.data_as(ctypes.c_void_p)))
                buf[:n].tofile(f)
                done += n
        else:
            done = 0
            while done < total:
                n = min(CHUNK, total - done)
                if fill == "zero":
                    chunk = np.zeros(n, np.float32)
                elif fill == "const":
                    chunk = np.full(n, value, np.float32)
                else:
                    chunk = np.arange(done, done + n, dtype=np.float64).astype(np.float32)
                chunk.tofile(f)
                done += n
    return path


def peek(uri, shape):
    path = file_path(uri)
    mm = np.memmap(path, np.float32, "r", shape=tuple(shape))
    if len(shape) == 1:
        n = shape[0]
        coords = [(0,), (n // 2,), (max(n - 1, 0),)]
    elif len(shape) == 2:
        r, c = shape
        coords = [(0, 0), (0, c - 1), (r // 2, c // 2), (r - 1, 0), (r - 1, c - 1)]
    else:
        raise JobError("peek supports rank <= 2")
    return [(co, float(mm[co])) for co in coords]


def main(argv=None):
    import argparse
    argv = sys.argv[1:] if argv is None else argv
    if not argv or argv[0] in ("-h", "--help"):
        print(USAGE)
        return 0
    cmd, rest = argv[0], argv[1:]
    ap = argparse.ArgumentParser(prog=f"python -m phobos_amd.tensor {cmd}")
    ap.add_argument("--uri", required=True)
    ap.add_argument("--shape", required=True)
    if cmd == "init":
        ap.add_argument("--fill", default="zero")
        ap.add_argument("--value", type=float, default=0.0)
        ap.add_argument("--seed", type=int, default=1)
    elif cmd != "peek":
        print(f"unknown subcommand '{cmd}'\n{USAGE}", file=sys.stderr)
        return 2
    a = ap.parse_args(rest)
    try:
        shape = parse_shape(a.shape)
        if cmd == "init":
            path = init(a.uri, shape, a.fill, a.value, a.seed)
            total = int(np.prod(shape))
            print(f"wrote {a.uri} ({total} elements, {total * 4} bytes, fill={a.fill}) to {path}")
        else:
            print(f"{a.uri} {shape}:")
            for co, v in peek(a.uri, shape):
                print(f"  [{','.join(map(str, co))}] = {v}")
    except (JobError, OSError) as e:
        print(f"error: {e}", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
