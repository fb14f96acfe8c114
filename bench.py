"""KV-cache PD-transfer benchmark on one MI355X.

Default: BASELINE.json configuration 2 (the headline). Llama-3-8B shape, 32
layers, 8 KV heads x 128, bf16 K and V (N(0,1) values generated on the
device), 64 requests x 2,048 tokens = 131,072 tokens = 16 GiB of KV. Source:
page_size-1 NHD pool of 262,144 slots with randomly permuted slots.
Destination: page_size-64 NHD pool with a random page table. Both pools and
the 16 GiB transfer buffer ([layer][K|V][token][head][dim]) are resident in
HBM before timing.

One step = pack every layer (pool -> transfer buffer) and unpack every layer
(transfer buffer -> decode pool): algorithmic bytes per step = 4 x payload
(pack reads + writes it, unpack reads + writes it again). The timed region
is bracketed by device synchronisation and carries no event between
launches; per-launch durations (roofline, per-layer p50) come from a second
pass over the same steps with HIP events on the launch stream around every
launch.

--config c1|c3|c4|c4fp8 runs the other co-resident configurations the same
way; --config c5 runs the ragged radix-prefix transfer in request waves
through the layer pipeline with its pinned-host hop (D2H then H2D), which
bounds it by the host link rather than HBM.

--config ceilings prints what plain contiguous streams reach on the device
(copy, read, write, hipMemcpyDtoD): the practical ceilings against which the
copy kernels' fractions of the nominal 8 TB/s should be read.

--config attn|attn_hnd measures the reader of the unpacked pages instead:
paged-attention decode over the C2 decode pool (NHD or head-major pages),
64 queries x 32 heads over 64 x 2,048 tokens, one launch per layer; its
line carries its own metric (GB/s of K/V read). --config attn_mla does the
same over the C4 pool in DeepSeek-V3's MLA form (K 576 / V 512 pair rows,
128 query heads on one KV head); --config attn64 reads the C2 page table
with head dims 64 (Llama-3.2-1B: 16 layers, 8 KV heads, 32 query heads;
attn64_hnd over head-major pages) and
--config attn256 with head dims 256 (Qwen3.5's full-attention layers: 2 KV
heads, 8 query heads; 16 layers).

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
ATTN_METRIC = "paged-attention decode GB/s of K/V read and % of HBM peak, Llama-3-8B shape"
MLA_METRIC = "paged-attention decode GB/s of K/V read and % of HBM peak, DeepSeek-V3 MLA shape"
ATTN64_METRIC = "paged-attention decode GB/s of K/V read and % of HBM peak, Llama-3.2-1B shape"
ATTN256_METRIC = "paged-attention decode GB/s of K/V read and % of HBM peak, Qwen3.5 head-dim-256 shape"
DIRECT_METRIC = "KV pool-to-pool transfer GB/s (bytes read + written) and % of HBM peak, Llama-3-8B shape"

DESCRIPTIONS = {
    "c1": "C1: Qwen2-0.5B-like GQA KV transfer, 24 layers x 2 KV heads x 64, bf16, 8 requests "
          "U[100,1000] tokens; src page_size-1 NHD pool of 65536 slots, dst page_size-16 NHD pool "
          "with a random page table",
    "c2": "C2: Llama-3-8B-shape GQA KV transfer, 32 layers x 8 KV heads x 128, bf16, 64 requests x "
          "2048 tokens (131072 tokens, 16 GiB KV); src page_size-1 NHD pool of 262144 slots, dst "
          "page_size-64 NHD pool with a random page table",
    "c3": "C3: one TP rank of Llama-3-70B (80 layers x 1 KV head x 128, bf16, 256-byte rows), 128 "
          "requests U[512,8192]; src page_size-1 NHD pool, dst page_size-64 HND pool",
    "c4": "C4: DeepSeek-V3/GLM-style MLA latent rows (61 layers x 576 bf16), 32 requests x 8192; "
          "src and dst page_size-64 pools with independent random page tables",
    "c4fp8": "C4 fp8: MLA latent rows as 576-byte fp8-e4m3 rows with per-layer scales passed "
             "through, 61 layers, 32 requests x 8192, page_size-64 -> page_size-64",
    "c4pair": "C4 over the pool the DeepSeek-V3 adapter allocates (models/deepseek.rs:360-369): "
              "61 layers of a tensor pair, 576-wide bf16 key (latent + rope, 1152 B) and 512-wide "
              "bf16 value (1024 B) per token, one launch per layer for both tensors; 32 requests x "
              "8192, page_size-64 -> page_size-64 with independent random page tables",
    "c4packed": "C4 over packed-MLA rows (packed_mla(61, 512, 64) = 649 bytes per token per "
                "layer, kv_cache.rs:201-224, models/deepseek.rs:1035-1037), byte-realigning "
                "kernels; 32 requests x 8192, page_size-64 -> page_size-64 with independent "
                "random page tables",
    "hnd64": "head chunks under 128 bytes: Llama-3.2-1B's KV shape (16 layers x 8 KV heads x 64) "
             "in fp8, 512-byte rows of eight 64-byte head chunks, 64 requests x 2048 tokens; src "
             "page_size-1 NHD pool of 262144 slots, dst page_size-64 HND pool with a random page "
             "table (head-major pages written in 64-byte pieces)",
    "nhd64": "as hnd64 with a page_size-64 NHD destination (whole 512-byte rows), the comparison "
             "for hnd64",
    "c2pages": "C2 shape as the reference transfers it today: page-for-page copies between "
               "page_size-64 pools of equal layout (131072 tokens = 2048 pages of 8 MiB, random "
               "source and destination pages), built with sgl_kv_build_page_requests and run "
               "as one launch (no relayout); algorithmic bytes = 2 x payload",
    "attn": "paged-attention decode over the C2 decode pool (the reader of the unpacked pages): "
            "Llama-3-8B shape, 32 layers x 8 KV heads x 128, bf16, page_size-64 NHD pool with a "
            "random page table, 64 requests x 2048 tokens, one decode query each with 32 query heads",
    "attn_hnd": "paged-attention decode as attn, over head-major (HND) pages",
    "attn64": "paged-attention decode with head dims 64 over the C2 decode pool's page table: "
              "Llama-3.2-1B shape, 16 layers x 8 KV heads x 64, bf16, page_size-64 NHD pool with "
              "a random page table, 64 requests x 2048 tokens, one decode query each with 32 "
              "query heads",
    "attn64_hnd": "paged-attention decode as attn64, over head-major (HND) pages (the layout the unpack "
                  "writes for a relayouting decode pool)",
    "attn256": "paged-attention decode with head dims 256 over the C2 decode pool's page table: "
               "Qwen3.5 full-attention shape (the reference's qwen3_5 config: 2 KV heads x 256, "
               "8 query heads), 16 layers, bf16, page_size-64 NHD pool with a random page table, "
               "64 requests x 2048 tokens, one decode query each",
    "attn_mla": "paged-attention decode over the C4 decode pool as DeepSeek-V3's MLA decode reads "
                "it: 61 layers of the reference's tensor-pair layout (576-wide latent+rope key, "
                "512-wide latent value, bf16, one KV head), page_size 64 with a random page "
                "table, 32 requests x 8192 tokens, one decode query each with 128 query heads",
    "ceilings": "the device's streaming ceilings: contiguous copy, read and write of 1 GiB in "
                "16-byte non-temporal vectors (sgl_rocm_kv_stream), hipMemcpyDtoD, the same copy "
                "over 16 GiB, and the host link (1 GiB DMA copies to and from pinned host memory, "
                "one direction at a time)",
    "c2direct": "C2 moved pool -> pool (sgl_rocm_kv_transfer_layer per layer, no transfer rows): "
                "the co-resident form of the C2 transfer; algorithmic bytes = 2 x payload",
    "c5": "C5: ragged radix-prefix GQA transfer (Llama-3-8B shape), 512 requests log-uniform "
          "[16,32768], page-aligned cached prefixes U[0,0.9]; request waves through the layer "
          "pipeline pack -> D2H -> pinned host -> H2D -> unpack on 4 streams",
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _traffic_from_profiles(kernel: str, summary: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary profiles/<summary>_counters.txt (FETCH_SIZE + WRITE_SIZE,
    calibrated), or None."""
    path = os.path.join(ROOT, "profiles", f"{summary}_counters.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"\s*traffic\s+(\S+)\s+bytes_per_launch=(\d+)", line)
        if m and m.group(1) == kernel:
            return int(m.group(2))
    return None


def cpu_baseline(make, seconds: float = 10.0, rows: int | None = 8192, threads: int = 1,
                 direct: bool = False):
    """The CPU oracle's pack + unpack (direct: its pool -> pool transfer) on
    `threads` host threads (rows split evenly) on the first `rows` tokens of
    the workload (None: the whole workload), repeated for about `seconds`
    (at least once)."""
    import oracle
    from sgl_rocm_kv import workloads as wl
    t = make() if rows is None else wl.scaled(make(), rows, seed=1)
    sh = t.shape
    n, T = t.rows, sh.tensors
    rb = [sh.tensor_row_bytes(i) for i in range(T)] + [0]
    lrb = sh.layer_row_bytes
    rng = np.random.default_rng(0)
    # (the whole workload's source pool: one byte value written over every
    # page, so each page is backed by its own memory; byte values do not
    # change a copy's speed, but an array never written maps every page to
    # the kernel's one zero page, whose reads hit in cache)
    src = (np.full(t.src.byte_len(sh), 0xA5, np.uint8) if rows is None
           else rng.integers(0, 256, t.src.byte_len(sh), dtype=np.uint8))
    dst = np.zeros(t.dst.byte_len(sh), np.uint8)
    buf = np.zeros(sh.layers * n * lrb, np.uint8)
    pools = []
    for layer in range(sh.layers):
        def opool(spec):
            return oracle.Pool(spec.page_size, spec.page_stride(sh), spec.page_count,
                               spec.tensor_offsets(sh, layer), rb[0], T, sh.heads,
                               spec.head_layout == 1, rb[1] if T == 2 and rb[1] != rb[0] else 0)
        part = buf[layer * n * lrb:(layer + 1) * n * lrb]
        pools.append((opool(t.src), opool(t.dst), part[: n * rb[0]], part[n * rb[0]:] if T == 2 else None))
    def one_pass():
        if direct:
            for sp, dp, _, _ in pools:
                oracle.transfer(sp, src, t.src_slots, dp, dst, t.dst_slots, threads=threads)
            return
        for sp, dp, r0, r1 in pools:
            oracle.pack(sp, src, t.src_slots, r0, r1, rb[0], rb[1], threads=threads)
        for sp, dp, r0, r1 in pools:
            oracle.unpack(dp, dst, t.dst_slots, r0, r1, rb[0], rb[1], threads=threads)

    one_pass()   # untimed: faults every page of the lazily mapped buffers in
    reps, t0 = 0, time.perf_counter()
    while True:
        one_pass()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 1000:
            break
    gbs = (2 if direct else 4) * t.payload_bytes * reps / el / 1e9
    which = "all" if rows is None else "first"
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"{t.name.split(' (')[0]} shape, {which} {n} tokens ({sh.layers} layers, "
                      f"{t.payload_bytes >> 20} MiB payload), "
                      f"{'pool -> pool transfer' if direct else 'pack+unpack'} x {reps} in {el:.1f} s, "
                      f"oracle/kv_oracle.c, {threads} thread{'s' if threads > 1 else ''}"}


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _usable_cores() -> int:
    """Cores this process may run on (its affinity mask; the box's share)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def _host_ram_bytes() -> int:
    try:
        return os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_PHYS_PAGES")
    except (ValueError, OSError):
        return 0


def _views(kv, buf, spec, sh, layer, scale=None):
    return kv.pool_view(buf.ptr, buf.nbytes, page_size=spec.page_size,
                        page_stride_bytes=spec.page_stride(sh), page_count=spec.page_count,
                        tensor_offset=spec.tensor_offsets(sh, layer), row_bytes=sh.row_bytes,
                        tensor_count=sh.tensors, heads=sh.heads, head_layout=spec.head_layout,
                        scale=scale,
                        value_row_bytes=sh.tensor_row_bytes(1) if sh.tensors == 2 and
                        sh.tensor_row_bytes(1) != sh.row_bytes else 0)


class _Span:
    """A device range (ptr, nbytes), optionally keeping its owner alive."""

    def __init__(self, ptr: int, nbytes: int, owner=None):
        self.ptr, self.nbytes, self.owner = ptr, nbytes, owner

    def download(self, nbytes: int, offset: int = 0) -> np.ndarray:
        from sgl_rocm_kv import hip
        assert offset + nbytes <= self.nbytes, "download past the end of the range"
        out = np.empty(nbytes, dtype=np.uint8)
        hip.memcpy_async(out.ctypes.data, self.ptr + offset, nbytes, "d2h")
        hip.synchronize()
        return out


def _placed_pool(kv, k, spec, sh, probe_rows, candidates: int, probe_source=None):
    """The destination pool from the library's placement probe
    (sgl_rocm_kv_storage_allocate_placed): `candidates` allocations held at
    once, each probed by packing one layer's rows into `probe_rows` (scratch,
    overwritten) and timing their unpack back, the fastest kept and
    zero-filled; with `probe_source` (a pool view) each candidate is timed on
    a pool-to-pool transfer from it instead. The same build's unpack into a pool runs
    at one of two speeds on MI355X depending on where the allocation lands in
    physical memory; the probe costs ~4 ms per candidate, outside the timed
    steps."""
    nbytes = spec.byte_len(sh)
    view = _views(kv, _Span(0, nbytes), spec, sh, 0)
    storage, report = kv.RocmKvStorage.allocate_placed(k, nbytes, spec.page_stride(sh), view,
                                                       probe_rows, candidates, probe_source=probe_source)
    report["probe_us"] = [round(x, 2) for x in report["probe_us"]]
    b = storage.allocation()
    log(f"destination pool: {report['candidates']} placement candidates, probe unpack "
        f"{report['probe_us']} us over {report['probe_rows']} rows, kept #{report['chosen']}")
    return _Span(b.ptr, b.byte_len, storage), report


def _kernel_family(sh):
    """The copy kernels a shape's rows take: the 16-byte-vector kernels when
    every row width is a whole number of 16-byte vectors (every address and
    stride of these workloads is then 16-byte aligned), the byte-realigning
    kernels otherwise (the 649-byte packed-MLA rows)."""
    if all(sh.tensor_row_bytes(t) % 16 == 0 for t in range(sh.tensors)):
        return "sglkv_copy_pool_rows_v16", "sglkv_copy_rows_pool_v16"
    return "sglkv_realign_pool_rows", "sglkv_realign_rows_pool"


def _pool_row_ranges(spec, sh, layer, slot):
    """(offset, length) pieces of (slot, layer)'s rows in a pool, tensor by
    tensor and head chunk by head chunk (the page-major layout of
    kv_cache.rs:653-700; HND pages keep each head's chunks together)."""
    page, pos = divmod(int(slot), spec.page_size)
    out = []
    for t, off in enumerate(spec.tensor_offsets(sh, layer)):
        rb = sh.tensor_row_bytes(t)
        region = page * spec.page_stride(sh) + off
        if spec.head_layout == 1:
            c = rb // sh.heads
            out += [(region + (h * spec.page_size + pos) * c, c) for h in range(sh.heads)]
        else:
            out.append((region + pos * rb, rb))
    return out


def verify_sample(t, src, xfer, dst, row_planes, rows_per_layer=64, seed=5):
    """After the timed steps: for a sample of rows on the first, middle and
    last layers, the source pool's bytes at the row's source slot, the
    packed transfer row and the destination pool's bytes at its destination
    slot must agree byte for byte (a check of the measured run itself; the
    parity tests compare with the CPU oracle). Returns rows checked."""
    sh = t.shape
    L = sh.layers
    rng = np.random.default_rng(seed)
    checked = 0
    for layer in sorted({0, L // 2, L - 1}):
        for r in rng.choice(t.rows, size=min(rows_per_layer, t.rows), replace=False):
            r = int(r)
            want = b"".join(bytes(src.download(n, o)) for o, n in
                            _pool_row_ranges(t.src, sh, layer, t.src_slots[r]))
            got_dst = b"".join(bytes(dst.download(n, o)) for o, n in
                               _pool_row_ranges(t.dst, sh, layer, t.dst_slots[r]))
            packed = b"".join(bytes(xfer.download(sh.tensor_row_bytes(tt), row_planes(layer, tt, r)))
                              for tt in range(sh.tensors))
            if not (want == packed == got_dst):
                raise SystemExit(f"verification failed: layer {layer} row {r} "
                                 f"(src slot {t.src_slots[r]}, dst slot {t.dst_slots[r]})")
            checked += 1
    return checked


def run_coresident(t, config, args):
    """Pack + unpack of every layer with both pools resident (C1-C4)."""
    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    sh = t.shape
    n, L, T = t.rows, sh.layers, sh.tensors
    rb = [sh.tensor_row_bytes(i) for i in range(T)]
    lrb = sh.layer_row_bytes           # one token's bytes in one layer, all tensors
    fp8 = config == "c4fp8"
    k = kv.RocmKvPairCopyKernels(0)
    src = hip.DeviceBuffer(t.src.byte_len(sh))
    xfer = hip.DeviceBuffer(L * n * lrb)
    dst, placement = _placed_pool(kv, k, t.dst, sh, kv.device_buffer(xfer.ptr, xfer.nbytes), args.placement)
    kind = kv.FILL_BITS if sh.elt_bytes == 1 else kv.FILL_BF16_NORMAL
    k.fill_synthetic(kv.device_buffer(src.ptr, src.nbytes), 2024, kind)
    k.fill_synthetic(kv.device_buffer(dst.ptr, dst.nbytes), 2025, kind)
    ss = hip.DeviceBuffer.from_array(t.src_slots)
    ds = hip.DeviceBuffer.from_array(t.dst_slots)
    ssb, dsb = kv.device_buffer(ss.ptr, ss.nbytes), kv.device_buffer(ds.ptr, ds.nbytes)
    scales = None
    if fp8:   # per-layer scales: source pool, transfer buffer, destination pool
        scales = [hip.DeviceBuffer.from_array(np.random.default_rng(i).random(L, dtype=np.float32))
                  for i in range(3)]
    hip.synchronize()
    log(f"pools resident: src {src.nbytes / 2**30:.1f} GiB, dst {dst.nbytes / 2**30:.1f} GiB, "
        f"transfer {xfer.nbytes / 2**30:.1f} GiB")

    def sc(i, layer):
        return scales[i].ptr + 4 * layer if scales else None

    # The transfer buffer is [layer][tensor][token][row bytes of the tensor].
    plane_off = [0] + [n * rb[0]] * (T - 1)

    def row_planes(layer, tt, r):
        return layer * n * lrb + plane_off[tt] + r * rb[tt]

    sviews = [_views(kv, src, t.src, sh, l, sc(0, l)) for l in range(L)]
    dviews = [_views(kv, dst, t.dst, sh, l, sc(2, l)) for l in range(L)]
    rviews = []
    for layer in range(L):
        base = xfer.ptr + layer * n * lrb
        rviews.append(kv.rows_view([base + plane_off[i] for i in range(T)], [n * rb[i] for i in range(T)],
                                   rb, sc(1, layer)))

    # All layers' rows as one view (multi-layer launches): plane t spans the
    # rest of the transfer buffer.
    all_rows = kv.rows_view([xfer.ptr + plane_off[i] for i in range(T)],
                            [xfer.nbytes - plane_off[i] for i in range(T)], rb, sc(1, 0))
    s_pack = hip.Stream()
    s_unpack = hip.Stream() if args.streams == 2 else s_pack
    auto = args.launch == "auto"
    if auto:   # measured on MI355X: per-layer launches win on large layers
        args.launch = "layers" if 2 * n * lrb < (256 << 20) else "layer"
    multi = args.launch == "layers"
    units = 1 if multi else L   # launches of each kind per step
    # Events for every launch of every instrumented step, read after the last
    # step, so that the device never idles between steps.
    ev = [[[hip.Event() for _ in range(4)] for _ in range(units)] for _ in range(args.steps)]
    gate = [hip.Event() for _ in range(units)]
    pool_stride_s = t.src.page_size * lrb
    pool_stride_d = t.dst.page_size * lrb

    def step(e_step):
        for u in range(units):
            e = e_step[u] if e_step else None
            if e:
                e[0].record(s_pack)
            if multi:
                k.pack_layers(sviews[0], pool_stride_s, L, ssb, n, all_rows, n * lrb, s_pack)
            else:
                k.pack_layer(sviews[u], ssb, n, rviews[u], s_pack)
            (e[1] if e else gate[u]).record(s_pack)
            if s_unpack is not s_pack:
                s_unpack.wait(e[1] if e else gate[u])
            if e:
                e[2].record(s_unpack)
            if multi:
                k.unpack_layers(all_rows, n * lrb, L, n, dviews[0], pool_stride_d, dsb, s_unpack)
            else:
                k.unpack_layer(rviews[u], n, dviews[u], dsb, s_unpack)
            if e:
                e[3].record(s_unpack)

    for _ in range(args.warmup):
        step(None)
    hip.synchronize()
    k.check_errors()
    log(f"warmup done ({args.warmup} steps, {'one launch per kind' if multi else 'per-layer launches'})")

    # Phase 1 (value): the timed steps carry no event between launches (an
    # event marker between kernels costs ~4 % of bandwidth on MI355X).
    hip.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(None)
    hip.synchronize()
    wall = time.perf_counter() - t0
    k.check_errors()
    log(f"timed {args.steps} steps in {wall:.3f} s")
    # Phase 2 (per-launch durations, per-layer p50): the same steps with an
    # event pair around every launch on its stream.
    for i in range(args.steps):
        step(ev[i])
    hip.synchronize()
    k.check_errors()
    pack_ms, unpack_ms, layer_us = [], [], []   # per layer
    kernel_ms = 0.0                              # all launches of all timed steps
    for e_step in ev:
        for e in e_step:
            p_ms, u_ms = e[0].elapsed_ms(e[1]), e[2].elapsed_ms(e[3])
            kernel_ms += p_ms + u_ms
            pack_ms.append(p_ms / (L if multi else 1))
            unpack_ms.append(u_ms / (L if multi else 1))
            layer_us.append((p_ms + u_ms) * 1e3 / (L if multi else 1))
    checked = verify_sample(t, src, xfer, dst, row_planes)
    log(f"verified {checked} sampled rows of the measured run (source = transfer row = destination)")

    if args.calibration_copy:
        span = min(1 << 30, xfer.nbytes // 2)
        for _ in range(3):
            hip.memcpy_async(xfer.ptr + span, xfer.ptr, span, "d2d", s_pack)
        s_pack.synchronize()
        log(f"calibration copies done (3 x {span} B device-to-device)")

    # The device's contiguous-copy ceiling, measured in the same process on
    # the transfer buffer (1 GiB each way; skipped for buffers too small to
    # stream past the caches).
    ceiling = None
    span = min(1 << 30, xfer.nbytes // 2)
    if span >= 256 << 20:
        a_buf = kv.device_buffer(xfer.ptr, span)
        b_buf = kv.device_buffer(xfer.ptr + span, span)
        for _ in range(3):
            k.stream_ceiling(kv.STREAM_COPY, a_buf, b_buf, span, s_pack)
        c0, c1 = hip.Event(), hip.Event()
        c0.record(s_pack)
        for _ in range(10):
            k.stream_ceiling(kv.STREAM_COPY, a_buf, b_buf, span, s_pack)
        c1.record(s_pack)
        c1.synchronize()
        ceiling = 2 * span * 10 / (c0.elapsed_ms(c1) / 1e3) / 1e9
        log(f"contiguous copy ceiling on this device: {ceiling:.0f} GB/s")

    step_bytes = t.algorithmic_bytes
    gbs = step_bytes / (wall / args.steps) / 1e9
    launch_bytes = n * lrb * 2        # one layer; pack_ms / unpack_ms are per layer
    avg_pack, avg_unpack = float(np.mean(pack_ms)), float(np.mean(unpack_ms))
    kernel_gbs = step_bytes / (kernel_ms / args.steps / 1e3) / 1e9
    pack_name, unpack_name = _kernel_family(sh)
    dom_name, dom_ms = ((pack_name, avg_pack) if avg_pack >= avg_unpack else (unpack_name, avg_unpack))
    achieved = launch_bytes / (dom_ms / 1e3) / 1e9
    log(f"pack avg {avg_pack * 1e3:.1f} us ({launch_bytes / avg_pack / 1e6:.0f} GB/s), "
        f"unpack avg {avg_unpack * 1e3:.1f} us ({launch_bytes / avg_unpack / 1e6:.0f} GB/s), "
        f"kernel-sum {kernel_gbs:.0f} GB/s, wall {gbs:.0f} GB/s")
    del src, dst, xfer
    k.close()
    payload_dtype = ("packed_mla_bytes" if config == "c4packed" else "fp8_e4m3" if sh.elt_bytes == 1
                     else "bf16")
    extra = {"tokens": n, "layers": L, "kv_heads": sh.heads, "head_dim": sh.head_dim,
             "row_bytes": rb, "payload_dtype": payload_dtype,
             "payload_bytes": t.payload_bytes, "algorithmic_bytes_per_step": step_bytes,
             "streams": args.streams, "launch": args.launch}
    return {
        "value": round(gbs, 1),
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "config_extra": extra,
        "per_layer_p50_us": round(float(np.percentile(layer_us, 50)), 2),
        "copy_ceiling": None if ceiling is None else {
            "gbs": round(ceiling, 1), "value_frac_of_ceiling": round(gbs / ceiling, 4),
            "note": "sgl_rocm_kv_stream contiguous copy of 1 GiB, same process: the most any "
                    "read+write stream reaches on this device"},
        "pack_us_avg": round(avg_pack * 1e3, 2),
        "unpack_us_avg": round(avg_unpack * 1e3, 2),
        "kernel_sum_gbs": round(kernel_gbs, 1),
        "verified_rows": checked,
        "placement": placement,
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     # the committed counter summaries were taken with --launch auto
                     "traffic": _traffic_from_profiles(dom_name, f"kv_copy_{config}") if auto else None,
                     "algorithmic_bytes_per_launch": launch_bytes * (L if multi else 1)},
    }


def run_staged(t, args):
    """C5: request waves through the layer pipeline with the pinned-host hop."""
    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    from sgl_rocm_kv import workloads as wl
    sh = t.shape
    rb, L, T = sh.row_bytes, sh.layers, sh.tensors
    max_rows, max_pages = 262144, 4096
    waves = wl.waves(t, max_rows, max_pages, seed=7)
    log(f"{len(waves)} waves; src pool {max_rows} slots, dst pool {max_pages} pages")
    k = kv.RocmKvPairCopyKernels(0)
    spec_s, spec_d = waves[0].src, waves[0].dst
    src = hip.DeviceBuffer(spec_s.byte_len(sh))
    dst = hip.DeviceBuffer(spec_d.byte_len(sh))
    k.fill_synthetic(kv.device_buffer(src.ptr, src.nbytes), 2024, kv.FILL_BF16_NORMAL)
    k.fill_synthetic(kv.device_buffer(dst.ptr, dst.nbytes), 2025, kv.FILL_BF16_NORMAL)
    layer_bytes = T * max(w.rows for w in waves) * rb
    send = [hip.DeviceBuffer(layer_bytes) for _ in range(2)]
    recv = [hip.DeviceBuffer(layer_bytes) for _ in range(2)]
    host = [hip.PinnedBuffer(layer_bytes) for _ in range(2)]
    sviews = [_views(kv, src, spec_s, sh, l) for l in range(L)]
    dviews = [_views(kv, dst, spec_d, sh, l) for l in range(L)]
    slot_bufs = [(hip.DeviceBuffer.from_array(w.src_slots), hip.DeviceBuffer.from_array(w.dst_slots))
                 for w in waves]
    hip.synchronize()

    def build(staged):
        return [kv.LayerPipeline(k, sviews, dviews, kv.device_buffer(a.ptr, a.nbytes),
                                 kv.device_buffer(b.ptr, b.nbytes), w.rows, send,
                                 recv if staged else None, host if staged else None)
                for w, (a, b) in zip(waves, slot_bufs)]

    def run_all(pipes):
        kernel_ms, hop_ms, lat = 0.0, [0.0, 0.0], []
        t0 = time.perf_counter()
        for p in pipes:
            p.run()
            p.wait()
        wall = time.perf_counter() - t0
        for p in pipes:
            for layer in range(L):
                pk, d2h, h2d, up, latency = p.layer_times(layer)
                kernel_ms += pk + up
                hop_ms[0] += d2h
                hop_ms[1] += h2d
                lat.append(latency * 1e3)
        return wall, kernel_ms, hop_ms, lat

    staged = build(True)
    direct = build(False)
    staged[0].run()     # warm-up: first wave once
    staged[0].wait()
    direct[0].run()
    direct[0].wait()
    log("warmup done")
    walls = []
    for _ in range(args.steps):
        wall, kernel_ms, hop_ms, lat = run_all(staged)
        walls.append(wall)
    dwall, dkernel_ms, _, _ = run_all(direct)
    for p in staged + direct:
        p.close()
    moved = t.payload_bytes
    wall = float(np.median(walls))
    gbs = 4 * moved / wall / 1e9
    kernel_gbs = 4 * moved / (kernel_ms / 1e3) / 1e9
    log(f"staged: {wall:.3f} s for {moved / 1e9:.1f} GB moved; host link {moved / wall / 1e9:.1f} "
        f"GB/s; D2H {moved / (hop_ms[0] / 1e3) / 1e9:.1f} GB/s, H2D {moved / (hop_ms[1] / 1e3) / 1e9:.1f} "
        f"GB/s per copy; kernels {kernel_gbs:.0f} GB/s; direct pipeline {4 * moved / dwall / 1e9:.0f} GB/s")
    k.close()
    return {
        "value": round(gbs, 1),
        "ms_per_step": round(wall * 1e3, 3),
        "config_extra": {"tokens_moved": t.rows, "layers": L, "waves": len(waves),
                         "payload_bytes": moved, "algorithmic_bytes_per_step": 4 * moved,
                         "streams": 4},
        "per_layer_p50_us": round(float(np.percentile(lat, 50)), 2),
        "host_link_gbs": round(moved / wall / 1e9, 2),
        "d2h_gbs_per_copy": round(moved / (hop_ms[0] / 1e3) / 1e9, 2),
        "h2d_gbs_per_copy": round(moved / (hop_ms[1] / 1e3) / 1e9, 2),
        "kernel_sum_gbs": round(kernel_gbs, 1),
        "direct_pipeline_gbs": round(4 * moved / dwall / 1e9, 1),
        "roofline": {"bound": "pcie", "kernel": "pipeline (pack, hop, unpack)",
                     "achieved": round(moved / wall / 1e9, 2), "peak": 64.0, "unit": "GB/s",
                     "frac": round(moved / wall / 1e9 / 64.0, 4), "traffic": None,
                     "note": "end-to-end bound by the host link: payload bytes per second over "
                             "PCIe Gen5 x16 (64 GB/s per direction); kernels alone reach "
                             f"{kernel_gbs:.0f} GB/s of HBM"},
    }


def run_pages(args):
    """The reference's PD transfer (transfer.rs:1945-2090) on one GPU: whole
    pages of equal-layout pools, one page request per page, executed by one
    launch per step."""
    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    from sgl_rocm_kv import workloads as wl
    sh = wl.c2().shape
    P, pages_moved, pool_pages = 64, 2048, 4096
    spec = wl.PoolSpec(P, pool_pages)
    pb = spec.page_stride(sh)
    rng = np.random.default_rng(11)
    src_pages = rng.permutation(pool_pages)[:pages_moved]
    dst_pages = rng.permutation(pool_pages)[:pages_moved]
    k = kv.RocmKvPairCopyKernels(0)
    src, dst = hip.DeviceBuffer(spec.byte_len(sh)), hip.DeviceBuffer(spec.byte_len(sh))
    k.fill_synthetic(kv.device_buffer(src.ptr, src.nbytes), 2024, kv.FILL_BF16_NORMAL)
    # the decode side's dst_kv_ptrs = [pool base], dst_kv_indices = its pages
    reqs = kv.build_remote_page_requests(src.ptr, pb, pages_moved * P, P, src_pages, [dst.ptr],
                                         dst_pages.astype(np.int32), pb)
    rq = hip.DeviceBuffer.from_array(reqs)
    args_k = (kv.device_buffer(rq.ptr, rq.nbytes), len(reqs), pb, kv.device_buffer(src.ptr, src.nbytes),
              kv.device_buffer(dst.ptr, dst.nbytes), True)
    s = hip.Stream()
    for _ in range(args.warmup):
        k.execute_page_requests(*args_k, stream=s)
    s.synchronize()
    k.check_errors()
    a, b = hip.Event(), hip.Event()
    hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        k.execute_page_requests(*args_k, stream=s)
    hip.synchronize()
    wall = time.perf_counter() - t0
    a.record(s)
    k.execute_page_requests(*args_k, stream=s)
    b.record(s)
    s.synchronize()
    k.check_errors()
    launch_ms = a.elapsed_ms(b)
    payload = pages_moved * pb
    gbs = 2 * payload / (wall / args.steps) / 1e9
    achieved = 2 * payload / (launch_ms / 1e3) / 1e9
    log(f"page requests: {len(reqs)} x {pb >> 20} MiB, wall {gbs:.0f} GB/s, launch {launch_ms:.3f} ms")
    # The ceiling at this footprint: one contiguous copy of the same payload
    # between the same two pools (HBM streams more slowly over 16 GiB than
    # over 1 GiB).
    sb, db = kv.device_buffer(src.ptr, payload), kv.device_buffer(dst.ptr, payload)
    k.stream_ceiling(kv.STREAM_COPY, sb, db, payload, s)
    a.record(s)
    for _ in range(3):
        k.stream_ceiling(kv.STREAM_COPY, sb, db, payload, s)
    b.record(s)
    s.synchronize()
    k.check_errors()
    ceiling = 2 * payload * 3 / (a.elapsed_ms(b) / 1e3) / 1e9
    log(f"contiguous copy of the same {payload >> 30} GiB: {ceiling:.0f} GB/s")
    if args.calibration_copy:   # a plain copy of known size for the counter runs
        span = 1 << 30
        for _ in range(3):
            hip.memcpy_async(dst.ptr, src.ptr, span, "d2d", s)
        s.synchronize()
        log(f"calibration copies done (3 x {span} B device-to-device)")
    k.close()
    return {
        "value": round(gbs, 1),
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "config_extra": {"pages": pages_moved, "page_bytes": pb, "payload_bytes": payload,
                         "algorithmic_bytes_per_step": 2 * payload},
        "copy_ceiling": {"gbs": round(ceiling, 1), "value_frac_of_ceiling": round(gbs / ceiling, 4),
                         "note": "sgl_rocm_kv_stream contiguous copy of the same payload between "
                                 "the same pools, same process"},
        "roofline": {"bound": "hbm", "kernel": "sglkv_copy_requests", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _traffic_from_profiles("sglkv_copy_requests", "kv_copy_c2pages"),
                     "algorithmic_bytes_per_launch": 2 * payload},
    }


def run_direct(t, args):
    """C2 moved pool -> pool (sgl_rocm_kv_transfer_layer per layer): what
    co-resident pools need, with no transfer rows between the two copies.
    Algorithmic bytes = 2 x payload (each K/V row read once, written once)."""
    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    sh = t.shape
    rb, n, L, T = sh.row_bytes, t.rows, sh.layers, sh.tensors
    k = kv.RocmKvPairCopyKernels(0)
    src = hip.DeviceBuffer(t.src.byte_len(sh))
    k.fill_synthetic(kv.device_buffer(src.ptr, src.nbytes), 2024, kv.FILL_BF16_NORMAL)
    # Each destination candidate is probed with a pool-to-pool transfer from
    # the source pool's first layer (the source is only read).
    dst, placement = _placed_pool(kv, k, t.dst, sh, None, args.placement,
                                  probe_source=_views(kv, src, t.src, sh, 0))
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    ssb, dsb = kv.device_buffer(ss.ptr, ss.nbytes), kv.device_buffer(ds.ptr, ds.nbytes)
    sviews = [_views(kv, src, t.src, sh, l) for l in range(L)]
    dviews = [_views(kv, dst, t.dst, sh, l) for l in range(L)]
    s = hip.Stream()

    def step(ev):
        for l in range(L):
            if ev:
                ev[l][0].record(s)
            k.transfer_layer(sviews[l], ssb, n, dviews[l], dsb, s)
            if ev:
                ev[l][1].record(s)

    for _ in range(args.warmup):
        step(None)
    hip.synchronize()
    k.check_errors()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(None)
    hip.synchronize()
    wall = time.perf_counter() - t0
    ev = [[[hip.Event(), hip.Event()] for _ in range(L)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(ev[i])
    hip.synchronize()
    k.check_errors()
    layer_ms = [e[0].elapsed_ms(e[1]) for es in ev for e in es]
    payload = L * T * n * rb
    launch_bytes = 2 * T * n * rb
    gbs = 2 * payload / (wall / args.steps) / 1e9
    achieved = launch_bytes / (float(np.mean(layer_ms)) / 1e3) / 1e9
    log(f"pool -> pool: {float(np.mean(layer_ms)) * 1e3:.1f} us per layer ({achieved:.0f} GB/s), wall {gbs:.0f} GB/s")
    if args.calibration_copy:   # a plain copy of known size for the counter runs
        span = 1 << 30
        for _ in range(3):
            hip.memcpy_async(dst.ptr, src.ptr, span, "d2d", s)
        s.synchronize()
        log(f"calibration copies done (3 x {span} B device-to-device)")
    traffic = _traffic_from_profiles("sglkv_copy_pool_pool_v16", "kv_copy_c2direct")
    k.close()
    return {
        "value": round(gbs, 1),
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "config_extra": {"tokens": n, "layers": L, "payload_bytes": payload,
                         "algorithmic_bytes_per_step": 2 * payload},
        "per_layer_p50_us": round(float(np.percentile(layer_ms, 50)) * 1e3, 2),
        "placement": placement,
        "roofline": {"bound": "hbm", "kernel": "sglkv_copy_pool_pool_v16", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes_per_launch": launch_bytes},
    }


def run_chunked(t, config, args):
    """Pack + unpack of every layer in args.chunks pieces through one reused
    transfer region of n / chunks rows: each piece's rows are unpacked right
    after they are packed, while the 256 MiB Infinity Cache still holds
    them. A schedule for co-resident pools, not what a transfer between
    devices sees (there the rows travel through HBM to the link)."""
    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    sh = t.shape
    rb, n, L, T = sh.row_bytes, t.rows, sh.layers, sh.tensors
    chunks = args.chunks
    if n % chunks:
        raise SystemExit(f"--chunks {chunks} does not divide {n} rows")
    m = n // chunks
    k = kv.RocmKvPairCopyKernels(0)
    src, dst = hip.DeviceBuffer(t.src.byte_len(sh)), hip.DeviceBuffer(t.dst.byte_len(sh))
    xfer = hip.DeviceBuffer(T * m * rb)
    k.fill_synthetic(kv.device_buffer(src.ptr, src.nbytes), 2024, kv.FILL_BF16_NORMAL)
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    sviews = [_views(kv, src, t.src, sh, l) for l in range(L)]
    dviews = [_views(kv, dst, t.dst, sh, l) for l in range(L)]
    rows = kv.rows_view([xfer.ptr + i * m * rb for i in range(T)], [m * rb] * T, [rb] * T, None)
    sb = [kv.device_buffer(ss.ptr + c * m * 8, m * 8) for c in range(chunks)]
    db = [kv.device_buffer(ds.ptr + c * m * 8, m * 8) for c in range(chunks)]
    s = hip.Stream()

    def step(ev):
        for l in range(L):
            if ev:
                ev[l][0].record(s)
            for c in range(chunks):
                k.pack_layer(sviews[l], sb[c], m, rows, s)
                k.unpack_layer(rows, m, dviews[l], db[c], s)
            if ev:
                ev[l][1].record(s)

    for _ in range(args.warmup):
        step(None)
    hip.synchronize()
    k.check_errors()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(None)
    hip.synchronize()
    wall = time.perf_counter() - t0
    ev = [[[hip.Event(), hip.Event()] for _ in range(L)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(ev[i])
    hip.synchronize()
    k.check_errors()
    layer_ms = [e[0].elapsed_ms(e[1]) for es in ev for e in es]
    step_bytes = t.algorithmic_bytes
    gbs = step_bytes / (wall / args.steps) / 1e9
    layer_bytes = step_bytes // L
    achieved = layer_bytes / (float(np.mean(layer_ms)) / 1e3) / 1e9
    log(f"{chunks} pieces per layer ({T * m * rb >> 20} MiB of rows each): wall {gbs:.0f} GB/s")
    k.close()
    return {
        "value": round(gbs, 1),
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "config_extra": {"tokens": n, "layers": L, "chunks_per_layer": chunks,
                         "transfer_region_bytes": T * m * rb, "algorithmic_bytes_per_step": step_bytes},
        "per_layer_p50_us": round(float(np.percentile(layer_ms, 50)) * 1e3, 2),
        "roofline": {"bound": "hbm", "kernel": "sglkv_copy_pool_rows_v16+sglkv_copy_rows_pool_v16",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": layer_bytes,
                     "note": "one layer = its chunks' pack and unpack launches; rows are re-read "
                             "from the Infinity Cache"},
    }


def _attention_geometry(config: str):
    """(layers, kv_heads, dk, dv, page_size, query_heads, scale) of an
    attention bench configuration: the C2 decode pool read by Llama-3-8B's
    32 query heads, or the C4 pool in the reference's MLA tensor-pair form
    (key 576 = kv_lora_rank 512 + rope 64, value 512; `models/deepseek.rs:
    360-369`) read by DeepSeek-V3's 128 heads at its qk head dim (192)."""
    if config == "attn_mla":
        return 61, 1, 576, 512, 64, 128, 1.0 / np.sqrt(192)
    if config in ("attn64", "attn64_hnd"):  # Llama-3.2-1B
        return 16, 8, 64, 64, 64, 32, 1.0 / np.sqrt(64)
    if config == "attn256":  # Qwen3.5's full-attention layers (model_registry.rs:628-660)
        return 16, 2, 256, 256, 64, 8, 1.0 / np.sqrt(256)
    return 32, 8, 128, 128, 64, 32, 1.0 / np.sqrt(128)


def _attention_layout(kv, config: str, pages: int):
    L, H, dk, dv, P, _, _ = _attention_geometry(config)
    kb, vb = H * dk * 2, H * dv * 2
    rt = kv.KvCacheRuntimeLayout("bf16", P, L, H, dk, 2, L * (kb + vb), L * (kb + vb) * P)
    if dk == dv:
        return kv.PagedKvCacheLayout.new(rt, pages)
    return kv.PagedKvCacheLayout.new_with_tensor_pair(rt, pages, kb, vb)


def attention_cpu_baseline(seconds: float, config: str):
    """The float64 attention oracle (numpy) on a sample of the attention
    workload: 2 of its decode queries over 2,048-token sequences, one layer,
    on a host pool holding just those pages."""
    import oracle
    import sgl_rocm_kv as kv
    hnd = config in ("attn_hnd", "attn64_hnd")
    L, H, dk, dv, P, qh, scale = _attention_geometry(config)
    n, nq = 2048, 2
    D = dk
    layout = _attention_layout(kv, config, nq * n // P)
    rng = np.random.default_rng(3)
    pool = rng.integers(0, 1 << 16, layout.total_byte_len // 2, dtype=np.uint16)
    pool &= np.uint16(0xBFFF)   # finite bf16 values of magnitude < 2
    slots = rng.permutation(layout.slot_count).astype(np.uint64)[: nq * n]
    q = oracle.f32_to_bf16(rng.standard_normal(nq * qh * D).astype(np.float32)).reshape(nq, qh, D)
    plan = kv.PagedAttentionPlan.for_layer(layout, 0, nq, nq, nq * n, qh, scale,
                                           kv.HND if hnd else kv.NHD)
    def one():
        oracle.paged_attention(pool.view(np.uint8), q, np.arange(nq), [n] * nq,
                               np.arange(nq + 1) * n, slots, page_size=P,
                               page_stride=plan.page_stride_bytes,
                               key_offset=plan.key_in_page_offset,
                               value_offset=plan.value_in_page_offset, kv_heads=H, dk=dk, dv=dv,
                               scale=scale, slot_count=layout.slot_count, hnd=hnd)
    one()
    reps, t0 = 0, time.perf_counter()
    while True:
        one()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 1000:
            break
    kv_bytes = nq * n * H * (dk + dv) * 2
    return {"value": round(kv_bytes * reps / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{nq} decode queries x {n} tokens x {qh} heads, one layer "
                      f"({kv_bytes >> 20} MiB of K/V), x {reps} in {el:.1f} s, float64 numpy "
                      f"oracle (oracle.paged_attention), single thread"}


def run_attention(args, config: str):
    """Decode attention over every layer of a decode pool: one async launch
    per layer on one stream. attn/attn_hnd read the C2 pool (Llama-3-8B GQA),
    attn64 the C2 page table at Llama-3.2-1B's head dims 64 (16 layers),
    attn256 at Qwen3.5's head dims 256 (2 KV heads, 8 query heads),
    attn_mla the C4 pool in MLA tensor-pair form. Algorithmic bytes per
    launch = the K and V rows the queries attend (C2: 64 x 2048 tokens x
    2 x 2,048 B; MLA: 32 x 8192 tokens x (1,152 + 1,024) B) + queries +
    outputs; the 8 B/token slot list is excluded, as the copies' slot maps
    are."""
    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    from sgl_rocm_kv import workloads as wl
    hnd, mla = config in ("attn_hnd", "attn64_hnd"), config == "attn_mla"
    t = wl.c4() if mla else wl.c2()
    L, H, dk, dv, P, qh, scale = _attention_geometry(config)
    D = dk
    assert t.dst.page_size == P and (config in ("attn64", "attn64_hnd", "attn256") or t.shape.layers == L)
    nreq, n = len(t.lengths), int(t.lengths[0])
    layout = _attention_layout(kv, config, t.dst.page_count)
    k = kv.RocmKvPairCopyKernels(0)
    pool = hip.DeviceBuffer(layout.total_byte_len)
    k.fill_synthetic(kv.device_buffer(pool.ptr, pool.nbytes), 2025, kv.FILL_BF16_NORMAL)
    rng = np.random.default_rng(9)
    import oracle
    q = oracle.f32_to_bf16(rng.standard_normal(nreq * qh * dk).astype(np.float32))
    bufs = dict(queries=hip.DeviceBuffer.from_array(q),
                query_request_indices=hip.DeviceBuffer.from_array(np.arange(nreq, dtype=np.uint32)),
                query_sequence_lengths=hip.DeviceBuffer.from_array(t.lengths.astype(np.uint64)),
                request_slot_offsets=hip.DeviceBuffer.from_array(
                    np.concatenate([[0], np.cumsum(t.lengths)]).astype(np.uint64)),
                sequence_slots=hip.DeviceBuffer.from_array(t.dst_slots), pool=pool)
    outs = [hip.DeviceBuffer(nreq * qh * dv * 2) for _ in range(L)]
    plans = [kv.PagedAttentionPlan.for_layer(layout, l, nreq, nreq, len(t.dst_slots), qh,
                                             scale, kv.HND if hnd else kv.NHD,
                                             fast_weights=args.fast_weights)
             for l in range(L)]
    s = hip.Stream()
    hip.synchronize()
    log(f"pool resident: {pool.nbytes / 2**30:.1f} GiB, {'HND' if hnd else 'NHD'} pages")

    def step(ev):
        for l in range(L):
            if ev:
                ev[l][0].record(s)
            k.paged_attention_async(plans[l], max_sequence_length=n, stream=s, output=outs[l], **bufs)
            if ev:
                ev[l][1].record(s)

    for _ in range(args.warmup):
        step(None)
    k.check_errors(s)
    hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(None)
    hip.synchronize()
    wall = time.perf_counter() - t0
    k.check_errors(s)
    ev = [[[hip.Event(), hip.Event()] for _ in range(L)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(ev[i])
    hip.synchronize()
    k.check_errors(s)
    launch_ms = [e[0].elapsed_ms(e[1]) for es in ev for e in es]
    if args.calibration_copy:   # a plain copy of known size for the counter runs
        span = 1 << 30
        for _ in range(3):
            hip.memcpy_async(pool.ptr + span, pool.ptr, span, "d2d", s)
        s.synchronize()
        log(f"calibration copies done (3 x {span} B device-to-device)")
    launch_bytes = nreq * n * H * (dk + dv) * 2 + nreq * qh * (dk + dv) * 2
    launch_flops = 2 * nreq * n * qh * (dk + dv)
    avg = float(np.mean(launch_ms))
    achieved = launch_bytes / (avg / 1e3) / 1e9
    gbs = launch_bytes * L / (wall / args.steps) / 1e9
    log(f"attention avg {avg * 1e3:.1f} us per layer ({achieved:.0f} GB/s, "
        f"{launch_flops / avg / 1e9:.1f} TFLOP/s), wall {gbs:.0f} GB/s")
    k.close()
    latent = "sglkv_paged_attention_latent" if args.fast_weights else "sglkv_paged_attention_latent_exact"
    kernel = (latent + "+sglkv_paged_attention_combine_h" if mla
              else ("sglkv_paged_attention_staged64" if D == 64
                    else "sglkv_paged_attention_staged256" if D == 256
                    else "sglkv_paged_attention_staged128k" if hnd else "sglkv_paged_attention_staged128")
              + "+sglkv_paged_attention_combine")
    summary = "paged_attention_decode_" + ("mla" if mla else ("dims64_hnd" if hnd else "dims64") if D == 64
                                           else "hnd" if hnd else "dims256" if D == 256 else "nhd")
    extra = {"requests": nreq, "tokens_per_request": n, "layers": L, "kv_heads": H,
             "query_heads": qh, "key_dim": dk, "value_dim": dv, "page_size": P,
             "head_layout": "HND" if hnd else "NHD",
             "softmax_weights": "one bf16 (ATTN_FAST_WEIGHTS)" if args.fast_weights else "hi + lo bf16 (default)",
             "algorithmic_bytes_per_step": launch_bytes * L}
    return {
        "value": round(gbs, 1),
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "config_extra": extra,
        "per_layer_p50_us": round(float(np.percentile(launch_ms, 50)) * 1e3, 2),
        # q.k and p.v at bf16: 2 * (dk + dv) flops per token per query head.
        "mfma_tflops": round(launch_flops / (avg / 1e3) / 1e12, 1),
        # One launch = the attention kernel and its combine pass: the events
        # bracket both (one C-ABI call), so the pair is the measured unit.
        "roofline": {"bound": "hbm", "kernel": kernel,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _traffic_from_profiles(kernel, summary),
                     "algorithmic_bytes_per_launch": launch_bytes},
    }


def run_ceilings(args):
    """What plain contiguous streams reach on this device: the practical
    ceilings the copy kernels' roofline fractions should be read against
    (HBM moves reads faster than writes, so a copy tops out well below the
    nominal peak)."""
    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    n = 1 << 30
    k = kv.RocmKvPairCopyKernels(0)
    a, b = hip.DeviceBuffer(n), hip.DeviceBuffer(n)
    k.fill_synthetic(kv.device_buffer(a.ptr, a.nbytes), 1, kv.FILL_BITS)
    k.fill_synthetic(kv.device_buffer(b.ptr, b.nbytes), 2, kv.FILL_BITS)
    ab, bb = kv.device_buffer(a.ptr, a.nbytes), kv.device_buffer(b.ptr, b.nbytes)
    s = hip.Stream()
    out = {}
    for name, launch, moved in (
            ("copy", lambda: k.stream_ceiling(kv.STREAM_COPY, ab, bb, n, s), 2 * n),
            ("read", lambda: k.stream_ceiling(kv.STREAM_READ, ab, bb, n, s), n),
            ("write", lambda: k.stream_ceiling(kv.STREAM_WRITE, None, bb, n, s), n),
            ("memcpy_dtod", lambda: hip.memcpy_async(b.ptr, a.ptr, n, "d2d", s), 2 * n)):
        for _ in range(args.warmup):
            launch()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(s)
        for _ in range(args.steps):
            launch()
        e1.record(s)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / args.steps
        out[name] = (moved / (ms / 1e3) / 1e9, ms)
        log(f"{name}: {ms * 1e3:.1f} us per GiB pass, {out[name][0]:.0f} GB/s")
    # The host link (what bounds C5): one direction at a time, runtime DMA
    # copies of 1 GiB between HBM and pinned host memory.
    host = hip.PinnedBuffer(n)
    for name, launch in (("link_d2h", lambda: hip.memcpy_async(host.ptr, a.ptr, n, "d2h", s)),
                         ("link_h2d", lambda: hip.memcpy_async(a.ptr, host.ptr, n, "h2d", s))):
        launch()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(s)
        for _ in range(3):
            launch()
        e1.record(s)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / 3
        out[name] = (n / (ms / 1e3) / 1e9, ms)
        log(f"{name}: {ms:.1f} ms per GiB, {out[name][0]:.1f} GB/s")
    # Both directions at once (what the C5 pipeline asks of the link): a
    # device-to-host and a host-to-device copy of 1 GiB on two streams,
    # three of each; each direction's rate over its own span, from events
    # on its stream.
    host2 = hip.PinnedBuffer(n)
    s2 = hip.Stream()
    hip.memcpy_async(host.ptr, a.ptr, n, "d2h", s)
    hip.memcpy_async(b.ptr, host2.ptr, n, "h2d", s2)
    s.synchronize()
    s2.synchronize()
    d0, d1, h0, h1 = hip.Event(), hip.Event(), hip.Event(), hip.Event()
    d0.record(s)
    h0.record(s2)
    for _ in range(3):
        hip.memcpy_async(host.ptr, a.ptr, n, "d2h", s)
        hip.memcpy_async(b.ptr, host2.ptr, n, "h2d", s2)
    d1.record(s)
    h1.record(s2)
    d1.synchronize()
    h1.synchronize()
    for name, ev0, ev1 in (("link_both_d2h", d0, d1), ("link_both_h2d", h0, h1)):
        ms = ev0.elapsed_ms(ev1) / 3
        out[name] = (n / (ms / 1e3) / 1e9, ms)
        log(f"{name} (both directions at once): {ms:.1f} ms per GiB, {out[name][0]:.1f} GB/s")
    host2.free()
    host.free()
    # The same copy over 16 GiB: HBM reaches a lower rate once the footprint
    # is far larger than the last-level cache, which is the regime of
    # transfers that move the whole pool in one launch (c2pages).
    a.free()
    b.free()
    big = 16 << 30
    a, b = hip.DeviceBuffer(big), hip.DeviceBuffer(big)
    abig, bbig = kv.device_buffer(a.ptr, big), kv.device_buffer(b.ptr, big)
    k.stream_ceiling(kv.STREAM_COPY, abig, bbig, big, s)
    e0, e1 = hip.Event(), hip.Event()
    e0.record(s)
    for _ in range(3):
        k.stream_ceiling(kv.STREAM_COPY, abig, bbig, big, s)
    e1.record(s)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / 3
    out["copy_16gib"] = (2 * big / (ms / 1e3) / 1e9, ms)
    log(f"copy 16 GiB: {ms:.2f} ms per pass, {out['copy_16gib'][0]:.0f} GB/s")
    a.free()
    b.free()
    k.check_errors(s)
    k.close()
    gbs = out["copy"][0]
    return {
        "value": round(gbs, 1),
        "ms_per_step": round(out["copy"][1], 4),
        "config_extra": {"bytes_per_pass": n, "algorithmic_bytes_per_step": 2 * n},
        "read_gbs": round(out["read"][0], 1),
        "write_gbs": round(out["write"][0], 1),
        "memcpy_dtod_gbs": round(out["memcpy_dtod"][0], 1),
        "copy_16gib_gbs": round(out["copy_16gib"][0], 1),
        "link_d2h_gbs": round(out["link_d2h"][0], 1),
        "link_h2d_gbs": round(out["link_h2d"][0], 1),
        "link_both_d2h_gbs": round(out["link_both_d2h"][0], 1),
        "link_both_h2d_gbs": round(out["link_both_h2d"][0], 1),
        "copy_engines": "blit kernels (HSA_ENABLE_SDMA=0)" if os.environ.get("HSA_ENABLE_SDMA") == "0"
                        else "SDMA engines (runtime default)",
        "roofline": {"bound": "hbm", "kernel": "sglkv_stream_copy", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": None, "algorithmic_bytes_per_launch": 2 * n},
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 20; C5: 1)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2", choices=sorted(DESCRIPTIONS))
    ap.add_argument("--streams", type=int, default=1, choices=(1, 2),
                    help="1: pack(l), unpack(l) in order on one stream (default: measured faster on "
                         "MI355X); 2: unpack of layer l on a second stream, overlapping pack of l+1")
    ap.add_argument("--launch", default="auto", choices=("auto", "layer", "layers"),
                    help="layer: one pack and one unpack launch per layer; layers: one launch of "
                         "each covering every layer; auto (default): layers when one layer moves "
                         "less than 256 MiB (launch-bound sizes), else layer")
    ap.add_argument("--chunks", type=int, default=1,
                    help="c2/c3/c4: pack and unpack each layer in this many pieces through one reused "
                         "transfer region (co-resident schedule; rows re-read from the Infinity Cache). "
                         "Default 1: whole layers, every layer's rows in its own region")
    ap.add_argument("--placement", type=int, default=3,
                    help="c1-c4, hnd64, nhd64, c2direct: allocate the destination pool this many times "
                         "at once, time one layer's unpack into each and keep the fastest "
                         "(sgl_rocm_kv_storage_allocate_placed; 1 = a single allocation, still probed "
                         "and reported)")
    ap.add_argument("--cpu-seconds", type=float, default=6.0,
                    help="seconds of CPU work per CPU-baseline figure")
    ap.add_argument("--cpu-threads", type=int, default=_usable_cores(),
                    help="threads of the all-core CPU baseline (default: every core this process "
                         "may use)")
    ap.add_argument("--cpu-full", action="store_true",
                    help="time the all-core CPU baseline on the whole workload (when host RAM "
                         "holds both pools and the rows) instead of its first 8192 tokens")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--fast-weights", action="store_true",
                    help="attention configs: plans with ATTN_FAST_WEIGHTS (the MLA latent body rounds "
                         "each softmax weight to one bf16 instead of a hi + lo pair)")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="after timing, run 3 hipMemcpyDtoD copies of exactly 1 GiB: a plain copy "
                         "kernel of known size that calibrates rocprofv3's FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 1 if args.config == "c5" else 20

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}, WORLD_SIZE {world}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from sgl_rocm_kv import workloads as wl
    makers = {"c1": wl.c1, "c2": wl.c2, "c3": wl.c3, "c4": wl.c4,
              "c4fp8": lambda: wl.c4(fp8=True), "c4pair": wl.c4pair, "c4packed": wl.c4packed,
              "c5": wl.c5, "c2pages": wl.c2, "attn": wl.c2,
              "hnd64": wl.chunks64, "nhd64": lambda: wl.chunks64(head_major=False),
              "attn_hnd": wl.c2, "attn_mla": wl.c4, "attn64": wl.c2, "attn64_hnd": wl.c2, "attn256": wl.c2, "ceilings": wl.c2,
              "c2direct": wl.c2}
    attention = args.config in ("attn", "attn_hnd", "attn_mla", "attn64", "attn64_hnd", "attn256")
    t = makers[args.config]()
    log(f"workload {t.name}: {t.rows} tokens moved, payload {t.payload_bytes / 2**30:.2f} GiB")
    if args.config == "c5":
        r = run_staged(t, args)
    elif args.config == "c2pages":
        r = run_pages(args)
    elif attention:
        r = run_attention(args, args.config)
    elif args.config == "ceilings":
        r = run_ceilings(args)
    elif args.config == "c2direct":
        r = run_direct(t, args)
    elif args.chunks > 1:
        if args.config not in ("c2", "c3", "c4"):
            raise SystemExit("--chunks applies to c2, c3 and c4")
        r = run_chunked(t, args.config, args)
    else:
        r = run_coresident(t, args.config, args)
    gbs = r.pop("value")
    extra = r.pop("config_extra")
    out = {
        "metric": ((MLA_METRIC if args.config == "attn_mla" else ATTN64_METRIC if args.config in ("attn64", "attn64_hnd")
                    else ATTN256_METRIC if args.config == "attn256" else ATTN_METRIC) if attention
                   else DIRECT_METRIC if args.config == "c2direct" else METRIC),
        "value": gbs,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if attention else "u8",
        "data": "synthetic (values generated on the device; seeded slot permutations and page tables)",
        "config": dict({"workload": DESCRIPTIONS[args.config], "parallelism": "single GPU"}, **extra),
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
    }
    out.update(r)
    out["cpu_baseline"] = None
    if args.config == "ceilings":
        out["metric"] = "device streaming ceilings: contiguous copy GB/s (read, write alongside)"
    elif not args.no_cpu_baseline:
        log("cpu baseline (oracle, 1 thread)")
        direct = args.config == "c2direct"
        out["cpu_baseline"] = (attention_cpu_baseline(args.cpu_seconds, args.config)
                               if attention else cpu_baseline(makers[args.config], args.cpu_seconds,
                                                              direct=direct))
        if not attention and args.cpu_threads > 1:
            # Every usable host core, beside the single-thread figure: on the
            # whole workload with --cpu-full when host RAM holds it, else on
            # the same sample.
            full = False
            if args.cpu_full:
                need = t.src.byte_len(t.shape) + t.dst.byte_len(t.shape) + t.payload_bytes
                full = need < _host_ram_bytes() // 2
                if not full:
                    log(f"--cpu-full: {need >> 30} GiB would not fit half of host RAM; sampling")
            log(f"cpu baseline (oracle, {args.cpu_threads} threads, {'full' if full else 'sample'})")
            out["cpu_baseline_all_cores"] = cpu_baseline(makers[args.config], args.cpu_seconds,
                                                         rows=None if full else 8192,
                                                         threads=args.cpu_threads, direct=direct)
        out["cpu_baseline"]["host_cores"] = _usable_cores()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
