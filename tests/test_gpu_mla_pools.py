"""GPU parity on the MLA pools the reference allocates, through the C ABI:

  - the DeepSeek-V3 adapter's tensor pair, a 576-wide key and a 512-wide
    value per token per layer (KvCacheModelLayout::tensor_pair(61, 1, 576, 1,
    512), crates/sglang-srt/src/models/deepseek.rs:360-369): 1,152 + 1,024
    bytes in bf16, moved in one launch per layer for both tensors, page size
    64 -> 64 and 64 -> 1, per layer, multi-layer, pool to pool, through the
    layer pipeline and through the transfer backend;
  - packed-MLA rows of 649 bytes (KvCacheModelLayout::packed_mla(61, 512,
    64), kv_cache.rs:201-224, models/deepseek.rs:1035-1037): odd row widths
    and strides through the byte-realigning kernels;
  - random unequal pair widths, odd widths and strides, HND chunks of odd
    size.

Expected bytes come from the CPU oracle (oracle/kv_oracle.c) with pool
geometry taken from the oracle's own layout functions
(ora_pair_tensor_token_byte_range, ora_tensor_token_byte_range), never from
the product's PagedKvCacheLayout.
"""
import numpy as np
import pytest

import oracle
import sgl_rocm_kv as kv
from sgl_rocm_kv import hip
from sgl_rocm_kv import workloads as wl

pytestmark = pytest.mark.gpu

LAYERS = 61


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


class Pools:
    """One side's pool described twice: by the product (for_model, pool
    views) and by the oracle (its own layout arithmetic)."""

    def __init__(self, model, dtype, widths, P, pages, per_layer_bytes):
        self.P, self.pages, self.widths = P, pages, widths
        self.layout = kv.PagedKvCacheLayout.for_model(model, dtype, P, P * pages)
        bpt = LAYERS * per_layer_bytes
        self.olay = oracle.layout(P, LAYERS, len(widths), bpt, P * bpt, pages)
        self.page_stride = P * bpt
        self.bytes = pages * P * bpt
        assert self.layout.total_byte_len == self.bytes

    def oracle_pool(self, layer):
        if len(self.widths) == 2:
            kb, vb = self.widths
            offs = [oracle.pair_tensor_token_byte_range(self.olay, kb, vb, 0, layer, t, 0)[1][0]
                    for t in range(2)]
            return oracle.Pool(self.P, self.page_stride, self.pages, tuple(offs), kb, 2, 1, False,
                               vb if vb != kb else 0)
        rc, (off, _) = oracle.tensor_token_byte_range(self.olay, 0, layer, 0, 0)
        assert rc == 0
        return oracle.Pool(self.P, self.page_stride, self.pages, (off,), self.widths[0], 1, 1, False)

    def view(self, buf, layer):
        return self.layout.pool_view(buf.ptr, buf.nbytes, layer)


def _pair(P, pages, fp8=False):
    elt = 1 if fp8 else 2
    model = kv.KvCacheModelLayout.tensor_pair(LAYERS, 1, 576, 1, 512)
    return Pools(model, "fp8_e4m3" if fp8 else "bf16", (576 * elt, 512 * elt), P, pages,
                 (576 + 512) * elt)


def _packed(P, pages):
    model = kv.KvCacheModelLayout.packed_mla(LAYERS, 512, 64)
    return Pools(model, "fp8_e4m3", (649,), P, pages, 649)


def _slots(rng, lengths, P, pages):
    """Slots of requests whose tokens fill random pages in order (the
    scheduler's page-contiguous allocation, model_executor.rs:158-175)."""
    _, _, slots = wl._page_table_slots(rng, np.asarray(lengths), np.zeros(len(lengths), int), P, pages)
    return slots


def _pages_for(lengths, P):
    return sum(-(-int(n) // P) for n in lengths)


def _rows_views(buf, n, widths, strides, layer_stride=0, layer=0):
    planes, off = [], layer * layer_stride
    for w, s in zip(widths, strides):
        planes.append(off)
        off += (n - 1) * s + w
    return kv.rows_view([buf.ptr + p for p in planes], [buf.nbytes - p for p in planes], list(strides)), planes


@pytest.mark.parametrize("dst_page_size", [64, 1])
def test_deepseek_pair_pool_every_layer(k, dst_page_size):
    """The DeepSeek-V3 pair pool, all 61 layers: pack each layer's key and
    value rows (one launch per layer), unpack into a decode pool of page size
    64 or 1, against the oracle on the same bytes."""
    _say(f"deepseek pair pool, 61 layers, P64 -> P{dst_page_size}")
    rng = np.random.default_rng(41 + dst_page_size)
    lengths = [1000, 777, 300]
    n = sum(lengths)
    sp = _pair(64, _pages_for(lengths, 64) + 5)
    dp = _pair(dst_page_size, _pages_for(lengths, dst_page_size) + 7)
    ss = _slots(rng, lengths, 64, sp.pages)
    ds = _slots(rng, lengths, dst_page_size, dp.pages)
    src_h = rng.integers(0, 256, sp.bytes, dtype=np.uint8)
    dst_h = rng.integers(0, 256, dp.bytes, dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    sb, dbf = hip.DeviceBuffer.from_array(ss), hip.DeviceBuffer.from_array(ds)
    kb, vb = sp.widths
    per_layer = n * (kb + vb)
    rows = hip.DeviceBuffer(LAYERS * per_layer)
    for layer in range(LAYERS):
        rv, _ = _rows_views(rows, n, (kb, vb), (kb, vb), per_layer, layer)
        k.pack_layer(sp.view(src, layer), _db(sb), n, rv)
        k.unpack_layer(rv, n, dp.view(dst, layer), _db(dbf))
    k.check_errors()
    want_rows = np.zeros(LAYERS * per_layer, np.uint8)
    want_dst = dst_h.copy()
    for layer in range(LAYERS):
        part = want_rows[layer * per_layer:(layer + 1) * per_layer]
        r0, r1 = part[: n * kb], part[n * kb:]
        oracle.pack(sp.oracle_pool(layer), src_h, ss, r0, r1, kb, vb, threads=8)
        oracle.unpack(dp.oracle_pool(layer), want_dst, ds, r0, r1, kb, vb, threads=8)
    np.testing.assert_array_equal(rows.download(), want_rows)
    np.testing.assert_array_equal(dst.download(), want_dst)

    # The same layers in one multi-layer launch of each kind, and pool to
    # pool, into fresh destinations.
    rows2 = hip.DeviceBuffer(LAYERS * per_layer)
    dst2 = hip.DeviceBuffer.from_array(dst_h)
    rv0, _ = _rows_views(rows2, n, (kb, vb), (kb, vb))
    k.pack_layers(sp.view(src, 0), sp.layout.bytes_per_layer_page, LAYERS, _db(sb), n, rv0, per_layer)
    k.unpack_layers(rv0, per_layer, LAYERS, n, dp.view(dst2, 0), dp.layout.bytes_per_layer_page, _db(dbf))
    dst3 = hip.DeviceBuffer.from_array(dst_h)
    k.transfer_layers(sp.view(src, 0), sp.layout.bytes_per_layer_page, LAYERS, _db(sb), n,
                      dp.view(dst3, 0), dp.layout.bytes_per_layer_page, _db(dbf))
    k.check_errors()
    np.testing.assert_array_equal(rows2.download(), want_rows)
    np.testing.assert_array_equal(dst2.download(), want_dst)
    np.testing.assert_array_equal(dst3.download(), want_dst)


@pytest.mark.parametrize("stride", [649, 656, 700, 651])
def test_packed_mla_rows(k, stride):
    """Packed-MLA rows (649 bytes, every row at a different alignment in the
    pool): pack into transfer rows of stride `stride`, unpack into a second
    packed pool, and pool to pool, every layer, against the oracle."""
    _say(f"packed-mla 649-byte rows, 61 layers, row stride {stride}")
    rng = np.random.default_rng(stride)
    lengths = [513, 1024, 64, 1]
    n = sum(lengths)
    sp, dp = _packed(64, _pages_for(lengths, 64) + 3), _packed(64, _pages_for(lengths, 64) + 9)
    ss, ds = _slots(rng, lengths, 64, sp.pages), _slots(rng, lengths, 64, dp.pages)
    src_h = rng.integers(0, 256, sp.bytes, dtype=np.uint8)
    dst_h = rng.integers(0, 256, dp.bytes, dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    sb, dbf = hip.DeviceBuffer.from_array(ss), hip.DeviceBuffer.from_array(ds)
    plane = (n - 1) * stride + 649
    rows = hip.DeviceBuffer(LAYERS * plane)
    rows.fill(0x5A)
    for layer in range(LAYERS):
        rv = kv.rows_view([rows.ptr + layer * plane], [plane], [stride])
        k.pack_layer(sp.view(src, layer), _db(sb), n, rv)
        k.unpack_layer(rv, n, dp.view(dst, layer), _db(dbf))
    k.check_errors()
    want_rows = np.full(LAYERS * plane, 0x5A, np.uint8)
    want_dst = dst_h.copy()
    for layer in range(LAYERS):
        r0 = want_rows[layer * plane:(layer + 1) * plane]
        oracle.pack(sp.oracle_pool(layer), src_h, ss, r0, None, stride, 0, threads=8)
        oracle.unpack(dp.oracle_pool(layer), want_dst, ds, r0, None, stride, 0, threads=8)
    np.testing.assert_array_equal(rows.download(), want_rows)
    np.testing.assert_array_equal(dst.download(), want_dst)
    dst2 = hip.DeviceBuffer.from_array(dst_h)
    k.transfer_layers(sp.view(src, 0), sp.layout.bytes_per_layer_page, LAYERS, _db(sb), n,
                      dp.view(dst2, 0), dp.layout.bytes_per_layer_page, _db(dbf))
    k.check_errors()
    np.testing.assert_array_equal(dst2.download(), want_dst)


def test_packed_mla_bad_slot_skips_only_its_row(k):
    """A slot past the pool on the realigning path: that row is skipped
    (its transfer row and its neighbours' bytes untouched), the others move,
    and the typed error is reported once."""
    rng = np.random.default_rng(7)
    sp = _packed(64, 4)
    n = 100
    ss = rng.permutation(sp.pages * 64)[:n].astype(np.uint64)
    ss[37] = sp.pages * 64 + 5
    src_h = rng.integers(0, 256, sp.bytes, dtype=np.uint8)
    src = hip.DeviceBuffer.from_array(src_h)
    sb = hip.DeviceBuffer.from_array(ss)
    plane = n * 649
    rows = hip.DeviceBuffer(plane)
    rows.fill(0xEE)
    k.pack_layer(sp.view(src, 3), _db(sb), n, kv.rows_view([rows.ptr], [plane], [649]))
    with pytest.raises(kv.KvError) as ei:
        k.check_errors()
    assert ei.value.variant == "DeviceSlotIndexOutOfRange"
    k.check_errors()  # consumed
    want = np.full(plane, 0xEE, np.uint8)
    good, _ = oracle.resolve_slots(sp.oracle_pool(3), n, slots=ss)
    oracle.pack(sp.oracle_pool(3), src_h, good, want, None, 649, 0)
    got = rows.download()
    assert (got[37 * 649:38 * 649] == 0xEE).all()
    np.testing.assert_array_equal(got, want)


def _random_realign_case(rng):
    """Random one- or two-tensor rows of widths that are mostly not whole
    16-byte vectors, NHD or HND (odd chunks), random strides and pages."""
    T = int(rng.integers(1, 3))
    H = int(rng.choice([1, 1, 2, 3, 5]))
    w = [H * int(rng.integers(1, 140)) for _ in range(T)]
    if T == 2 and rng.random() < 0.3:
        w[1] = w[0]
    rows = int(rng.choice([1, 7, 64, 333, 1500]))
    specs = []
    for _ in range(2):
        P = int(rng.choice([1, 3, 16, 64]))
        pages = -(-rows // P) + int(rng.integers(0, 3))
        specs.append((P, pages, int(rng.integers(0, 2)) if H > 1 else 0))
    strides = [wi + int(rng.choice([0, 0, 1, 3, 8, 17])) for wi in w]
    return T, H, w, rows, specs, strides


@pytest.mark.parametrize("seed", range(48))
def test_random_unequal_and_odd_widths(k, seed):
    """Random pair widths (unequal), odd widths and strides, HND chunks of
    odd size, page sizes 1-64: pack, unpack and pool to pool on one layer of
    a two-layer pool, against the oracle."""
    rng = np.random.default_rng(7000 + seed)
    T, H, w, n, specs, strides = _random_realign_case(rng)
    _say(f"realign case {seed}: T={T} H={H} widths={w} rows={n} pools={specs} strides={strides}")
    L, layer = 2, int(rng.integers(0, 2))
    lrb = sum(w)
    pools, kviews, host = [], [], []
    for P, pages, hnd in specs:
        page_stride = P * L * lrb
        offs = tuple(layer * P * lrb + t * P * w[0] for t in range(T))
        pools.append(oracle.Pool(P, page_stride, pages, offs, w[0], T, H, bool(hnd),
                                 w[1] if T == 2 and w[1] != w[0] else 0))
        h = rng.integers(0, 256, pages * page_stride, dtype=np.uint8)
        host.append(h)
    bufs = [hip.DeviceBuffer.from_array(h) for h in host]
    for (P, pages, hnd), b in zip(specs, bufs):
        kviews.append(kv.pool_view(b.ptr, b.nbytes, page_size=P, page_stride_bytes=P * L * lrb,
                                   page_count=pages,
                                   tensor_offset=[layer * P * lrb + t * P * w[0] for t in range(T)],
                                   row_bytes=w[0], tensor_count=T, heads=H, head_layout=hnd,
                                   value_row_bytes=w[1] if T == 2 and w[1] != w[0] else 0))
    ss = rng.permutation(specs[0][0] * specs[0][1])[:n].astype(np.uint64)
    ds = rng.permutation(specs[1][0] * specs[1][1])[:n].astype(np.uint64)
    sb, dbf = hip.DeviceBuffer.from_array(ss), hip.DeviceBuffer.from_array(ds)
    planes = [(n - 1) * s + wi for wi, s in zip(w, strides)]
    rows = hip.DeviceBuffer(sum(planes) + 3)
    rows.fill(0x11)
    base = rows.ptr + 3  # an odd plane base
    rv = kv.rows_view([base, base + planes[0]][:T], planes, strides)
    k.pack_layer(kviews[0], _db(sb), n, rv)
    k.unpack_layer(rv, n, kviews[1], _db(dbf))
    k.check_errors()
    want_rows = np.full(sum(planes) + 3, 0x11, np.uint8)
    r0 = want_rows[3:3 + planes[0]]
    r1 = want_rows[3 + planes[0]:] if T == 2 else None
    oracle.pack(pools[0], host[0], ss, r0, r1, strides[0], strides[-1])
    want_dst = host[1].copy()
    oracle.unpack(pools[1], want_dst, ds, r0, r1, strides[0], strides[-1])
    np.testing.assert_array_equal(rows.download(), want_rows)
    np.testing.assert_array_equal(bufs[1].download(), want_dst)
    # pool to pool into a fresh copy of the destination
    d2 = hip.DeviceBuffer.from_array(host[1])
    kview2 = kv.pool_view(d2.ptr, d2.nbytes, page_size=specs[1][0],
                          page_stride_bytes=specs[1][0] * L * lrb, page_count=specs[1][1],
                          tensor_offset=[layer * specs[1][0] * lrb + t * specs[1][0] * w[0]
                                         for t in range(T)],
                          row_bytes=w[0], tensor_count=T, heads=H, head_layout=specs[1][2],
                          value_row_bytes=w[1] if T == 2 and w[1] != w[0] else 0)
    k.transfer_layer(kviews[0], _db(sb), n, kview2, _db(dbf))
    k.check_errors()
    want2 = host[1].copy()
    oracle.transfer(pools[0], host[0], ss, pools[1], want2, ds)
    np.testing.assert_array_equal(d2.download(), want2)


@pytest.mark.parametrize("kind", ["pair", "packed"])
def test_staged_pipeline_on_mla_pools(k, kind):
    """The layer pipeline (pack -> pinned host -> unpack on four streams) on
    the pair pool and on the packed pool, all 61 layers, against the oracle."""
    _say(f"staged pipeline on the {kind} pool")
    rng = np.random.default_rng(99 if kind == "pair" else 98)
    lengths = [600, 129]
    n = sum(lengths)
    mk = _pair if kind == "pair" else _packed
    sp, dp = mk(64, _pages_for(lengths, 64) + 2), mk(16, _pages_for(lengths, 16) + 5)
    ss, ds = _slots(rng, lengths, 64, sp.pages), _slots(rng, lengths, 16, dp.pages)
    src_h = rng.integers(0, 256, sp.bytes, dtype=np.uint8)
    dst_h = rng.integers(0, 256, dp.bytes, dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    sb, dbf = hip.DeviceBuffer.from_array(ss), hip.DeviceBuffer.from_array(ds)
    layer_bytes = n * sum(sp.widths)
    send = [hip.DeviceBuffer(layer_bytes) for _ in range(2)]
    recv = [hip.DeviceBuffer(layer_bytes) for _ in range(2)]
    host = [hip.PinnedBuffer(layer_bytes) for _ in range(2)]
    pipe = kv.LayerPipeline(k, [sp.view(src, l) for l in range(LAYERS)],
                            [dp.view(dst, l) for l in range(LAYERS)], _db(sb), _db(dbf), n, send, recv, host)
    pipe.run()
    pipe.wait()
    pipe.close()
    want = dst_h.copy()
    for layer in range(LAYERS):
        oracle.transfer(sp.oracle_pool(layer), src_h, ss, dp.oracle_pool(layer), want, ds, threads=8)
    np.testing.assert_array_equal(dst.download(), want)


@pytest.mark.parametrize("mode", [kv.BACKEND_DIRECT, kv.BACKEND_STAGED])
def test_backend_moves_the_deepseek_pair_pool(k, mode):
    """The transfer backend registers the DeepSeek-V3 pair pools (keys 1,152
    and values 1,024 bytes) and moves spans with cached prefixes between
    them, against the oracle."""
    _say(f"backend on the deepseek pair pool, mode {mode}")
    rng = np.random.default_rng(123 + mode)
    sp, dp = _pair(64, 40), _pair(64, 48)
    src_h = rng.integers(0, 256, sp.bytes, dtype=np.uint8)
    dst_h = rng.integers(0, 256, dp.bytes, dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    be = kv.RocmKvTransferBackend(k, mode, max_rows=4096)
    be.register(sp.layout, src.ptr, src.nbytes, dp.layout, dst.ptr, dst.nbytes)
    want = dst_h.copy()
    free = list(rng.permutation(sp.pages))
    dfree = list(rng.permutation(dp.pages))
    for room, (prefix, count) in enumerate([(0, 500), (128, 300), (64, 1)]):
        pages = [free.pop() for _ in range(-(-count // 64))]
        slots = np.concatenate([np.arange(p * 64, p * 64 + 64) for p in pages])[:count].astype(np.uint64)
        table = np.array([dfree.pop() for _ in range(-(-(prefix + count) // 64))], np.int32)
        be.submit(room, f"{room:064x}", prefix, slots, table)
        tok = prefix + np.arange(count)
        dslots = (table[tok // 64].astype(np.int64) * 64 + tok % 64).astype(np.uint64)
        for layer in range(LAYERS):
            oracle.transfer(sp.oracle_pool(layer), src_h, slots, dp.oracle_pool(layer), want, dslots)
    be.wait()
    events, pending = be.poll()
    assert pending == 0 and sorted(e.bootstrap_room for e in events) == [0, 1, 2]
    assert all(e.status == kv.TRANSFER_COMPLETED for e in events), events
    be.close()
    np.testing.assert_array_equal(dst.download(), want)


def test_backend_rejects_more_than_two_tensors(k):
    """A layout of three tensors per token is rejected at register, not
    moved partially."""
    rt = kv.KvCacheRuntimeLayout.for_model("bf16", 16, 2, 1, 64, 3)
    lay = kv.PagedKvCacheLayout.new(rt, 2)
    buf = hip.DeviceBuffer(lay.total_byte_len)
    be = kv.RocmKvTransferBackend(k, kv.BACKEND_DIRECT, max_rows=64)
    with pytest.raises(kv.KvError) as ei:
        be.register(lay, buf.ptr, buf.nbytes, lay, buf.ptr, buf.nbytes)
    assert ei.value.variant == "InvalidArgument" and ei.value.name == "kv_tensors_per_token"
    be.close()
