"""GPU checks of every benchmark configuration at its full size, through the
C ABI: the runs behind the bench lines, verified.

Each case fills the source pool on the device with the reproducible
splitmix64 stream (sgl_rocm_kv_fill_synthetic, FILL_BITS; its host copy
kv.synthetic_words is pinned to splitmix64's published outputs in
tests/test_host_abi.py), packs every layer, unpacks every layer into the
decode pool and packs every layer again from the decode pool. Then:

  - the packed rows of the first, middle and last layers equal the source
    words recomputed on the host at each row's source slot, for every row;
  - a random sample of rows of every other layer does too;
  - the destination pool itself, read back region by region with plain
    copies and addressed on the host: every row of the first, middle and
    last layers sits at its destination slot (NHD or HND) holding the
    source words, every other byte of those layers' regions in the pages
    the destination table names still holds the destination's own fill,
    and a seeded sample of 64 pages the table does not name is unchanged
    in full (on C2 these reads reach offsets past 2^32 bytes);
  - the re-packed rows equal the packed rows on every layer (the unpack
    placed every row where the destination slots say, as the re-pack reads
    them; the unpack itself is compared with the oracle on the same shapes
    at reduced size in tests/test_gpu_parity.py and test_gpu_mla_pools.py).

Source and destination byte addresses come from the workload's own
page-major arithmetic (workloads.PoolSpec, restating kv_cache.rs:653-700),
not from the product.

C5 runs its request waves (workloads.waves) through the staged layer
pipeline (pack -> pinned host -> unpack on four streams) and checks, wave by
wave, a sample of rows of every layer read back from the decode pool.
"""
import numpy as np
import pytest

import sgl_rocm_kv as kv
from sgl_rocm_kv import hip
from sgl_rocm_kv import workloads as wl

pytestmark = pytest.mark.gpu

SEED = 0xF1115


def _say(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def k():
    if hip.device_count() == 0:
        pytest.fail("no GPU visible: the gpu tests need an MI355X")
    ctx = kv.RocmKvPairCopyKernels(0)
    yield ctx
    ctx.close()


def _db(buf, offset=0, nbytes=None):
    return kv.device_buffer(buf.ptr + offset, buf.nbytes - offset if nbytes is None else nbytes)


def _view(buf, spec, sh, layer):
    return kv.pool_view(buf.ptr, buf.nbytes, page_size=spec.page_size,
                        page_stride_bytes=spec.page_stride(sh), page_count=spec.page_count,
                        tensor_offset=spec.tensor_offsets(sh, layer), row_bytes=sh.row_bytes,
                        tensor_count=sh.tensors, heads=sh.heads, head_layout=spec.head_layout,
                        value_row_bytes=sh.tensor_row_bytes(1) if sh.tensors == 2 and
                        sh.tensor_row_bytes(1) != sh.row_bytes else 0)


def _rows(buf, n, sh):
    rb = [sh.tensor_row_bytes(t) for t in range(sh.tensors)]
    offs = [0, n * rb[0]][:sh.tensors]
    return kv.rows_view([buf.ptr + o for o in offs], [buf.nbytes - o for o in offs], rb)


def _source_bytes(seed, spec, sh, layer, tensor, slots):
    """The bytes (len(slots) x row bytes) of an NHD source pool filled with
    the FILL_BITS stream of `seed`, at `slots` for (layer, tensor)."""
    rb = sh.tensor_row_bytes(tensor)
    s = np.asarray(slots, np.int64)
    page, pos = s // spec.page_size, s % spec.page_size
    start = page * spec.page_stride(sh) + spec.tensor_offsets(sh, layer)[tensor] + pos * rb
    nw = rb // 8 + 2
    idx = (start // 8)[:, None] + np.arange(nw, dtype=np.int64)[None, :]
    words = kv.synthetic_words(seed, idx.reshape(-1).astype(np.uint64)).reshape(len(s), nw)
    b = words.view(np.uint8).reshape(len(s), nw * 8)
    sel = (start % 8)[:, None] + np.arange(rb, dtype=np.int64)[None, :]
    return np.take_along_axis(b, sel, axis=1)


def _check_layer_rows(rows_buf, t, sh, layer, seed, sample=None, rng=None):
    """Packed rows of `layer` against the host-recomputed source bytes: every
    row, or `sample` random rows."""
    n, lrb = t.rows, sh.layer_row_bytes
    base = layer * n * lrb
    plane = 0
    for tensor in range(sh.tensors):
        rb = sh.tensor_row_bytes(tensor)
        if sample is None:
            for lo in range(0, n, 8192):
                hi = min(n, lo + 8192)
                got = rows_buf.download((hi - lo) * rb, base + plane + lo * rb).reshape(hi - lo, rb)
                want = _source_bytes(seed, t.src, sh, layer, tensor, t.src_slots[lo:hi])
                np.testing.assert_array_equal(got, want, err_msg=f"layer {layer} tensor {tensor} rows {lo}..{hi}")
        else:   # `sample` rows in blocks of 16 consecutive rows
            for lo in rng.choice(max(1, n - 16), size=max(1, sample // 16), replace=False):
                lo = int(lo)
                hi = min(n, lo + 16)
                got = rows_buf.download((hi - lo) * rb, base + plane + lo * rb).reshape(hi - lo, rb)
                want = _source_bytes(seed, t.src, sh, layer, tensor, t.src_slots[lo:hi])
                np.testing.assert_array_equal(got, want, err_msg=f"layer {layer} tensor {tensor} rows {lo}..{hi}")
        plane += n * rb


def _fill_bytes(seed, start, nbytes):
    """Bytes [start, start + nbytes) of a buffer filled with the FILL_BITS
    stream of `seed`."""
    w0 = start // 8
    nw = (start + nbytes + 7) // 8 - w0
    words = kv.synthetic_words(seed, np.arange(w0, w0 + nw, dtype=np.uint64))
    return words.view(np.uint8)[start - 8 * w0: start - 8 * w0 + nbytes]


def _check_destination(dst, t, sh, layer, label):
    """Every row of `layer` read straight from the destination pool at its
    destination slot (host arithmetic, head chunk by head chunk on HND
    pages), against the source words; every other byte of the layer's
    regions in the pages the rows touch against the destination fill.
    Returns the largest pool offset read."""
    spec, P = t.dst, t.dst.page_size
    region_bytes = P * sh.layer_row_bytes        # the layer's tensors, consecutive in a page
    region0 = spec.tensor_offsets(sh, layer)[0]
    dslots = np.asarray(t.dst_slots, np.int64)
    pages, where = np.unique(dslots // P, return_inverse=True)
    got = np.empty((len(pages), region_bytes), np.uint8)
    top = 0
    for i, page in enumerate(pages):
        off = int(page) * spec.page_stride(sh) + region0
        got[i] = dst.download(region_bytes, off)
        top = max(top, off + region_bytes)
    written = np.zeros_like(got, dtype=bool)
    pos = dslots % P
    for tensor in range(sh.tensors):
        rb = sh.tensor_row_bytes(tensor)
        toff = spec.tensor_offsets(sh, layer)[tensor] - region0
        chunks = sh.heads if spec.head_layout == kv.HND else 1
        c = rb // chunks
        for lo in range(0, t.rows, 16384):
            hi = min(t.rows, lo + 16384)
            want = _source_bytes(SEED, t.src, sh, layer, tensor, t.src_slots[lo:hi])
            for h in range(chunks):
                if spec.head_layout == kv.HND:
                    at = toff + (h * P + pos[lo:hi]) * c
                else:
                    at = toff + pos[lo:hi] * rb + h * c
                idx = at[:, None] + np.arange(c)[None, :]
                rows = where[lo:hi][:, None]
                np.testing.assert_array_equal(got[rows, idx], want[:, h * c:(h + 1) * c],
                                              err_msg=f"{label} layer {layer} tensor {tensor} head {h} rows {lo}..{hi}")
                written[rows, idx] = True
    # the rest of those regions: the destination's own fill, untouched
    for i, page in enumerate(pages):
        if written[i].all():
            continue
        off = int(page) * spec.page_stride(sh) + region0
        fill = _fill_bytes(SEED + 1, off, region_bytes)
        keep = ~written[i]
        assert np.array_equal(got[i][keep], fill[keep]), f"{label} layer {layer} page {page}: stray write"
    return top


def _check_untouched_pages(dst, t, sh, label, count=64, seed=17):
    """`count` seeded pages that no destination slot names, each compared in
    full with the destination's fill. Returns the largest offset read."""
    spec = t.dst
    used = np.unique(np.asarray(t.dst_slots, np.int64) // spec.page_size)
    free = np.setdiff1d(np.arange(spec.page_count), used)
    if not len(free):   # C4: 262,144 rows fill all 4,096 pages; the region checks cover them
        _say(f"{label}: the destination table names every page")
        return 0
    rng = np.random.default_rng(seed)
    top = 0
    for page in rng.choice(free, size=min(count, len(free)), replace=False):
        off = int(page) * spec.page_stride(sh)
        n = spec.page_stride(sh)
        assert np.array_equal(dst.download(n, off), _fill_bytes(SEED + 1, off, n)), \
            f"{label}: page {page} outside the destination table changed"
        top = max(top, off + n)
    return top


def _equal_on_host(a, b, nbytes, chunk=1 << 30):
    for off in range(0, nbytes, chunk):
        m = min(chunk, nbytes - off)
        if not np.array_equal(a.download(m, off), b.download(m, off)):
            return off
    return None


def _full_size(k, t, label):
    sh = t.shape
    n, L = t.rows, sh.layers
    lrb = sh.layer_row_bytes
    rows_bytes = L * n * lrb
    need = t.src.byte_len(sh) + t.dst.byte_len(sh) + 2 * rows_bytes + 16 * n
    free, _ = hip.mem_info()
    if free < need + (4 << 30):
        pytest.skip(f"needs {need >> 30} GiB of device memory, {free >> 30} GiB free")
    _say(f"{label} full size: {n} rows x {L} layers, {rows_bytes / 2**30:.1f} GiB of rows")
    src, dst = hip.DeviceBuffer(t.src.byte_len(sh)), hip.DeviceBuffer(t.dst.byte_len(sh))
    k.fill_synthetic(_db(src), SEED, kv.FILL_BITS)
    k.fill_synthetic(_db(dst), SEED + 1, kv.FILL_BITS)
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    packed, again = hip.DeviceBuffer(rows_bytes), hip.DeviceBuffer(rows_bytes)
    pa, pb = _rows(packed, n, sh), _rows(again, n, sh)
    sstride, dstride = t.src.page_size * lrb, t.dst.page_size * lrb
    k.pack_layers(_view(src, t.src, sh, 0), sstride, L, _db(ss), n, pa, n * lrb)
    k.unpack_layers(pa, n * lrb, L, n, _view(dst, t.dst, sh, 0), dstride, _db(ds))
    k.pack_layers(_view(dst, t.dst, sh, 0), dstride, L, _db(ds), n, pb, n * lrb)
    k.check_errors()
    del src
    rng = np.random.default_rng(3)
    full = sorted({0, L // 2, L - 1})
    for layer in range(L):
        if layer in full:
            _say(f"{label}: every row of layer {layer} against the source words")
            _check_layer_rows(packed, t, sh, layer, SEED)
        else:
            _check_layer_rows(packed, t, sh, layer, SEED, sample=64, rng=rng)
    top = 0
    for layer in full:
        _say(f"{label}: layer {layer} read straight from the destination pool")
        top = max(top, _check_destination(dst, t, sh, layer, label))
    _say(f"{label}: 64 pages outside the destination table")
    top = max(top, _check_untouched_pages(dst, t, sh, label))
    del dst
    _say(f"{label}: pack -> unpack -> re-pack on all {L} layers")
    bad = _equal_on_host(packed, again, rows_bytes)
    assert bad is None, f"re-packed rows differ in the GiB at byte {bad}"
    return top


def test_c2_full_size_every_layer(k):
    """C2: 131,072 rows x 32 layers (16 GiB of rows), P1 -> P64; the
    destination reads reach past 2^32 bytes of the 32 GiB pool."""
    top = _full_size(k, wl.c2(), "C2")
    assert top > 1 << 32


def test_c3_full_size_every_layer(k):
    """C3: 550,621 rows x 80 layers of 256-byte rows, P1 NHD -> P64 HND."""
    _full_size(k, wl.c3(), "C3")


@pytest.mark.parametrize("kind", ["c4", "c4fp8", "c4pair", "c4packed"])
def test_c4_full_size_every_layer(k, kind):
    """C4 in each of its forms at 262,144 rows x 61 layers: 576-wide bf16
    and fp8 rows, the DeepSeek-V3 key/value pair and the 649-byte packed
    rows, page size 64 on both sides."""
    t = {"c4": wl.c4, "c4fp8": lambda: wl.c4(fp8=True), "c4pair": wl.c4pair,
         "c4packed": wl.c4packed}[kind]()
    _full_size(k, t, kind.upper())


@pytest.mark.parametrize("kind", ["hnd64", "nhd64"])
def test_64_byte_head_chunks_full_size(k, kind):
    """The hnd64 / nhd64 bench configurations at 131,072 rows x 16 layers:
    fp8 rows of eight 64-byte head chunks into page_size-64 HND or NHD pages."""
    _full_size(k, wl.chunks64(head_major=kind == "hnd64"), kind.upper())


def test_c5_waves_through_the_staged_pipeline(k):
    """C5: the ragged radix-prefix transfer in the request waves the bench
    runs (workloads.waves over a 262,144-slot source pool and a 4,096-page
    decode pool), each through the staged layer pipeline; after every wave,
    a sample of rows of every layer is read back from the decode pool and
    compared with the source words at their source slots."""
    t = wl.c5()
    sh = t.shape
    L, rb = sh.layers, sh.row_bytes
    waves = wl.waves(t, 262144, 4096, seed=7)
    assert sum(w.rows for w in waves) == t.rows
    spec_s, spec_d = waves[0].src, waves[0].dst
    _say(f"C5: {len(waves)} waves, {t.rows} rows moved")
    src, dst = hip.DeviceBuffer(spec_s.byte_len(sh)), hip.DeviceBuffer(spec_d.byte_len(sh))
    k.fill_synthetic(_db(src), SEED, kv.FILL_BITS)
    k.fill_synthetic(_db(dst), SEED + 1, kv.FILL_BITS)
    layer_bytes = 2 * max(w.rows for w in waves) * rb
    send = [hip.DeviceBuffer(layer_bytes) for _ in range(2)]
    recv = [hip.DeviceBuffer(layer_bytes) for _ in range(2)]
    host = [hip.PinnedBuffer(layer_bytes) for _ in range(2)]
    sviews = [_view(src, spec_s, sh, l) for l in range(L)]
    dviews = [_view(dst, spec_d, sh, l) for l in range(L)]
    back = hip.DeviceBuffer(layer_bytes)
    rng = np.random.default_rng(11)
    for i, w in enumerate(waves):
        ss, ds = hip.DeviceBuffer.from_array(w.src_slots), hip.DeviceBuffer.from_array(w.dst_slots)
        pipe = kv.LayerPipeline(k, sviews, dviews, _db(ss), _db(ds), w.rows, send, recv, host)
        pipe.run()
        pipe.wait()
        pipe.close()
        _say(f"C5 wave {i}: {w.rows} rows, checking every layer")
        rv = _rows(back, w.rows, sh)
        blocks = [int(b) for b in rng.choice(max(1, w.rows - 32), size=8, replace=w.rows < 300)]
        for layer in range(L):
            k.pack_layer(dviews[layer], _db(ds), w.rows, rv)
            k.check_errors()
            for tensor in range(2):
                for lo in blocks:
                    hi = min(w.rows, lo + 32)
                    got = back.download((hi - lo) * rb, tensor * w.rows * rb + lo * rb).reshape(hi - lo, rb)
                    want = _source_bytes(SEED, spec_s, sh, layer, tensor, w.src_slots[lo:hi])
                    assert np.array_equal(got, want), f"wave {i} layer {layer} tensor {tensor} rows {lo}..{hi}"
