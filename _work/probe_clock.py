"""Shader clock and matrix-core occupancy of the f16 kernels at the BASELINE
shapes, measured from inside the kernels.

Measurement tool, not part of the library: it loads the PHX_CLOCK_PROBE code
objects that `make -C phobos-lang_amd probe` builds into lib/probe/.  In those
builds each workgroup (GEMM) or wave (flash) reads s_memtime (shader clock)
and s_memrealtime (100 MHz) at its start and end and writes both spans, /64,
over its first outputs, so the outputs are not attention or GEMM results.

    make -C phobos-lang_amd probe && python3 phobos-lang_amd/probe_clock.py

MFMA busy = the v_mfma_f32_32x32x16_f16 cycles a SIMD needs for its waves'
share of the work (32 cycles each) / the span in shader cycles.
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
os.environ["PHX_CODE_OBJECT_DIR"] = os.path.join(HERE, "lib", "probe")
sys.path.insert(0, HERE)

import numpy as np  # noqa: E402

import phobos_amd as px  # noqa: E402

N, BH, S, D = 4096, 64, 4096, 64
MFMA_CYCLES = 32


def report(name, cyc, rt_us, mfma_cycles):
    print(f"{name:22s} span {cyc.mean():9.0f} cycles = {rt_us.mean():7.1f} us -> shader clock "
          f"{(cyc / rt_us).mean():6.0f} MHz, MFMA busy {mfma_cycles / cyc.mean():.2f}", flush=True)


def main(reps=30):
    if not os.path.isdir(os.environ["PHX_CODE_OBJECT_DIR"]):
        sys.exit("build the probe code objects first: make -C phobos-lang_amd probe")
    px.init(0)
    s = px.Stream()
    a32 = px.from_f16_bits(px.to_f16_bits(px.normal_f32(1, N * N, 1 / 64.0)))
    b32 = px.from_f16_bits(px.to_f16_bits(px.normal_f32(2, N * N, 1 / 64.0)))
    for name, kid, a, b, esz in (("gemm_fp16tc_fp32acc", px.GEMM_FP16TC_FP32ACC, a32, b32, 4),
                                 ("gemm_fp16", px.GEMM_FP16, px.to_f16_bits(a32),
                                  px.to_f16_bits(b32), 2)):
        da, db = px.DeviceBuffer.from_array(a), px.DeviceBuffer.from_array(b)
        c = px.DeviceBuffer(N * N * esz)
        for _ in range(reps):
            px.launch_gemm(s, kid, da, db, c, N, N, N, 1.0, 0.0)
        s.synchronize()
        C = c.download(np.float32, (N, N)) if esz == 4 else \
            px.from_f16_bits(c.download(np.uint16, (N, N)))
        C = C.astype(np.float64) * 64  # first two outputs of every 256x256 tile
        # one wave per SIMD computes a 128x128 quarter: 4096/16 K slices x 16 MFMAs
        report(name, C[::256, ::256].ravel(), C[::256, 1::256].ravel() / 100,
               (N // 16) * 16 * MFMA_CYCLES)
    ts = [px.to_f16_bits(px.normal_f32(sd, BH * S * D)) for sd in (1, 2, 3)]
    q, k, v = (px.DeviceBuffer.from_array(t) for t in ts)
    o = px.DeviceBuffer(BH * S * D * 2)
    for _ in range(reps):
        px.launch_flash_bh(s, px.FLASH_FP16_BH, q, k, v, o, BH, S, S, D, 0.125)
    s.synchronize()
    O = px.from_f16_bits(o.download(np.uint16, (BH * S, D))).astype(np.float64) * 64
    # first query row of every 32-query wave; four waves share a SIMD, each
    # running 16 MFMAs per 64-key block
    report("flash_fp16", O[::32, 0], O[::32, 1] / 100, 4 * (S // 64) * 16 * MFMA_CYCLES)


if __name__ == "__main__":
    main()
