"""KV-cache PD-transfer benchmark on one MI355X.

Workload (Llama-3-8B shape): 32 layers, 8 KV heads x 128, bf16 K and V
(N(0,1) values generated on the device), 64 requests x 2,048 tokens =
131,072 tokens = 16 GiB of KV. Source: page_size-1 NHD pool of 262,144
slots with randomly permuted slots. Destination: page_size-64 NHD pool with
a random page table. Both pools and the 16 GiB transfer buffer
([layer][K|V][token][head][dim]) are resident in HBM before timing.

One step = pack every layer (pool -> transfer buffer) and unpack every layer
(transfer buffer -> decode pool): algorithmic bytes per step = 4 x payload
(pack reads + writes it, unpack reads + writes it again). The timed region
is bracketed by device synchronisation; per-launch durations come from HIP
events recorded on the launch stream inside the timed steps.

Prints one JSON line (the driver's contract), with a `roofline` object for
the dominant kernel and a `cpu_baseline` object: the CPU oracle
(oracle/kv_oracle.c, one thread) timed on a bounded sample of the same
workload on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "sglang-rs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "KV pack+unpack GB/s and % of HBM peak, Llama-3-8B shape; per-layer p50 µs"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _traffic_from_profiles(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, calibrated), or None."""
    path = os.path.join(ROOT, "profiles", "kv_copy_c2_counters.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"\s*traffic\s+(\S+)\s+bytes_per_launch=(\d+)", line)
        if m and m.group(1) == kernel:
            return int(m.group(2))
    return None


def cpu_baseline(seconds: float = 10.0, rows: int = 8192):
    """The CPU oracle's pack + unpack (1 thread) on the first `rows` tokens
    of the C2 workload, repeated for about `seconds`."""
    import oracle
    from sgl_rocm_kv import workloads as wl
    t = wl.scaled(wl.c2(), rows, seed=1)
    sh = t.shape
    rb, n = sh.row_bytes, t.rows
    rng = np.random.default_rng(0)
    src = rng.integers(0, 256, t.src.byte_len(sh), dtype=np.uint8)
    dst = np.zeros(t.dst.byte_len(sh), np.uint8)
    buf = np.zeros(sh.layers * 2 * n * rb, np.uint8)
    pools = []
    for layer in range(sh.layers):
        sp = oracle.Pool(1, t.src.page_stride(sh), t.src.page_count, t.src.tensor_offsets(sh, layer),
                         rb, 2, sh.heads, False)
        dp = oracle.Pool(t.dst.page_size, t.dst.page_stride(sh), t.dst.page_count,
                         t.dst.tensor_offsets(sh, layer), rb, 2, sh.heads, False)
        part = buf[layer * 2 * n * rb:(layer + 1) * 2 * n * rb]
        pools.append((sp, dp, part[: n * rb], part[n * rb:]))
    reps, t0 = 0, time.perf_counter()
    while True:
        for sp, dp, k_rows, v_rows in pools:
            oracle.pack(sp, src, t.src_slots, k_rows, v_rows, rb, rb, threads=1)
        for sp, dp, k_rows, v_rows in pools:
            oracle.unpack(dp, dst, t.dst_slots, k_rows, v_rows, rb, rb, threads=1)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 1000:
            break
    gbs = 4 * t.payload_bytes * reps / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"C2 shape, first {n} tokens (32 layers, {t.payload_bytes >> 20} MiB payload), "
                      f"pack+unpack x {reps} in {el:.1f} s, oracle/kv_oracle.c single thread"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--streams", type=int, default=1, choices=(1, 2),
                    help="1: pack(l), unpack(l) in order on one stream (default: measured faster on "
                         "MI355X); 2: unpack of layer l on a second stream, overlapping pack of l+1")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="after timing, run 3 hipMemcpyDtoD copies of exactly 1 GiB: a plain copy "
                         "kernel of known size that calibrates rocprofv3's FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}, WORLD_SIZE {world}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    from sgl_rocm_kv import workloads as wl

    t = wl.c2()
    sh = t.shape
    rb, n, L = sh.row_bytes, t.rows, sh.layers
    log(f"workload {t.name}: {n} tokens, payload {t.payload_bytes / 2**30:.1f} GiB")
    k = kv.RocmKvPairCopyKernels(0)
    src = hip.DeviceBuffer(t.src.byte_len(sh))
    dst = hip.DeviceBuffer(t.dst.byte_len(sh))
    xfer = hip.DeviceBuffer(L * 2 * n * rb)
    k.fill_synthetic(kv.device_buffer(src.ptr, src.nbytes), 2024, kv.FILL_BF16_NORMAL)
    k.fill_synthetic(kv.device_buffer(dst.ptr, dst.nbytes), 2025, kv.FILL_BF16_NORMAL)
    ss = hip.DeviceBuffer.from_array(t.src_slots)
    ds = hip.DeviceBuffer.from_array(t.dst_slots)
    ssb, dsb = kv.device_buffer(ss.ptr, ss.nbytes), kv.device_buffer(ds.ptr, ds.nbytes)
    hip.synchronize()
    log(f"pools resident: src {src.nbytes >> 30} GiB, dst {dst.nbytes >> 30} GiB, "
        f"transfer {xfer.nbytes >> 30} GiB")

    sviews, dviews, rviews = [], [], []
    for layer in range(L):
        sviews.append(kv.pool_view(src.ptr, src.nbytes, page_size=1,
                                   page_stride_bytes=t.src.page_stride(sh), page_count=t.src.page_count,
                                   tensor_offset=t.src.tensor_offsets(sh, layer), row_bytes=rb,
                                   tensor_count=2, heads=sh.heads))
        dviews.append(kv.pool_view(dst.ptr, dst.nbytes, page_size=t.dst.page_size,
                                   page_stride_bytes=t.dst.page_stride(sh), page_count=t.dst.page_count,
                                   tensor_offset=t.dst.tensor_offsets(sh, layer), row_bytes=rb,
                                   tensor_count=2, heads=sh.heads))
        base = xfer.ptr + layer * 2 * n * rb
        rviews.append(kv.rows_view([base, base + n * rb], [n * rb] * 2, [rb, rb]))

    s_pack = hip.Stream()
    s_unpack = hip.Stream() if args.streams == 2 else s_pack
    ev = [[hip.Event() for _ in range(4)] for _ in range(L)]

    def step(timed: bool):
        for layer in range(L):
            e = ev[layer]
            if timed:
                e[0].record(s_pack)
            k.pack_layer(sviews[layer], ssb, n, rviews[layer], s_pack)
            e[1].record(s_pack)
            if s_unpack is not s_pack:
                s_unpack.wait(e[1])
            if timed:
                e[2].record(s_unpack)
            k.unpack_layer(rviews[layer], n, dviews[layer], dsb, s_unpack)
            if timed:
                e[3].record(s_unpack)

    for _ in range(args.warmup):
        step(False)
    hip.synchronize()
    k.check_errors()
    log(f"warmup done ({args.warmup} steps)")

    pack_ms, unpack_ms, layer_us = [], [], []
    hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
        # Per-launch durations: read after each step so events are reused safely.
        s_pack.synchronize()
        s_unpack.synchronize()
        for layer in range(L):
            e = ev[layer]
            p_ms, u_ms = e[0].elapsed_ms(e[1]), e[2].elapsed_ms(e[3])
            pack_ms.append(p_ms)
            unpack_ms.append(u_ms)
            layer_us.append((p_ms + u_ms) * 1e3)
    hip.synchronize()
    wall = time.perf_counter() - t0
    k.check_errors()
    log(f"timed {args.steps} steps in {wall:.3f} s")

    step_bytes = t.algorithmic_bytes
    ms_per_step = wall * 1e3 / args.steps
    gbs = step_bytes / (wall / args.steps) / 1e9
    launch_bytes = 2 * n * rb * 2   # one layer: K+V rows read and written
    avg_pack, avg_unpack = float(np.mean(pack_ms)), float(np.mean(unpack_ms))
    kernel_gbs = step_bytes / ((sum(pack_ms) + sum(unpack_ms)) / args.steps / 1e3) / 1e9
    dom_name, dom_ms = (("sglkv_copy_pool_rows_v16", avg_pack) if avg_pack >= avg_unpack
                        else ("sglkv_copy_rows_pool_v16", avg_unpack))
    achieved = launch_bytes / (dom_ms / 1e3) / 1e9
    log(f"pack avg {avg_pack * 1e3:.1f} us ({launch_bytes / avg_pack / 1e6:.0f} GB/s), "
        f"unpack avg {avg_unpack * 1e3:.1f} us ({launch_bytes / avg_unpack / 1e6:.0f} GB/s), "
        f"kernel-sum {kernel_gbs:.0f} GB/s, wall {gbs:.0f} GB/s")

    out = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (bf16 N(0,1) generated on the device; seeded slot permutation and page table)",
        "config": {
            "workload": "C2: Llama-3-8B-shape GQA KV transfer, 32 layers x 8 KV heads x 128, bf16, "
                        "64 requests x 2048 tokens (131072 tokens, 16 GiB KV); src page_size-1 NHD "
                        "pool of 262144 slots, dst page_size-64 NHD pool with a random page table",
            "tokens": n, "layers": L, "kv_heads": sh.heads, "head_dim": sh.head_dim,
            "payload_dtype": "bf16", "payload_bytes": t.payload_bytes,
            "algorithmic_bytes_per_step": step_bytes, "streams": args.streams,
            "parallelism": "single GPU",
        },
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "per_layer_p50_us": round(float(np.percentile(layer_us, 50)), 2),
        "pack_us_avg": round(avg_pack * 1e3, 2),
        "unpack_us_avg": round(avg_unpack * 1e3, 2),
        "kernel_sum_gbs": round(kernel_gbs, 1),
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _traffic_from_profiles(dom_name),
                     "algorithmic_bytes_per_launch": launch_bytes},
        "cpu_baseline": None,
    }
    if args.calibration_copy:
        for _ in range(3):
            hip.memcpy_async(xfer.ptr + (1 << 30), xfer.ptr, 1 << 30, "d2d", s_pack)
        s_pack.synchronize()
        log("calibration copies done (3 x 1 GiB device-to-device)")
    del src, dst, xfer
    k.close()
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle, 1 thread)")
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
