"""GPU parity: every device entry point of libsgl_rocm_kv against the CPU
oracle (oracle/kv_oracle.c) on the same seeded input bytes, bit for bit.

Cases:
  - the reference's own acceptance test of the pair scatter/gather kernels
    (crates/sglang-srt/tests/cuda_backend.rs:497-637);
  - pack / unpack / pool-to-pool transfer on every benchmark shape (C1 at
    full size; C2-C5 on the first few thousand rows), NHD and HND pages,
    page sizes 1/16/64, MLA single-tensor rows, fp8 rows with per-layer
    scales, span + page-table resolution with cached prefixes;
  - edge cases: empty and single-row transfers, ragged tile tails,
    unaligned row strides (every vector width), out-of-range slots and page
    entries (typed errors, untouched bytes);
  - (every benchmark configuration at full size: tests/test_gpu_full_size.py).
"""
import numpy as np
import pytest

import oracle
import sgl_rocm_kv as kv
from sgl_rocm_kv import hip
from sgl_rocm_kv import workloads as wl

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def k():
    if hip.device_count() == 0:
        pytest.fail("no GPU visible: the gpu tests need an MI355X")
    ctx = kv.RocmKvPairCopyKernels(0)
    yield ctx
    ctx.close()


def _db(buf):
    return kv.device_buffer(buf.ptr, buf.nbytes)


def _opool(spec, shape, layer, hnd=None):
    return oracle.Pool(spec.page_size, spec.page_stride(shape), spec.page_count,
                       spec.tensor_offsets(shape, layer), shape.row_bytes, shape.tensors,
                       shape.heads, spec.head_layout == kv.HND if hnd is None else hnd)


def _kpool(buf, spec, shape, layer, scale=None):
    return kv.pool_view(buf.ptr, buf.nbytes, page_size=spec.page_size,
                        page_stride_bytes=spec.page_stride(shape), page_count=spec.page_count,
                        tensor_offset=spec.tensor_offsets(shape, layer), row_bytes=shape.row_bytes,
                        tensor_count=shape.tensors, heads=shape.heads, head_layout=spec.head_layout,
                        scale=scale)


# --- the reference acceptance test, through the drop-in pair API -------------------------------

def _acceptance(goldens):
    g = goldens["scatter_gather_acceptance"]
    rt = goldens["cuda_backend_slot_location"]["runtime"]
    runtime = kv.KvCacheRuntimeLayout(rt["dtype"], rt["page_size"], rt["num_layers"], rt["kv_heads"],
                                      rt["head_dim"], rt["kv_tensors_per_token"], rt["bytes_per_token"],
                                      rt["page_size_bytes"])
    return g, kv.PagedKvCacheLayout.new(runtime, g["page_count"])


def test_reference_acceptance_scatter_then_gather(k, goldens):
    """cuda_kv_kernels_scatter_and_gather_batched_physical_slots: slots
    1, 15, 16, 31 across a page boundary, strided rows (+37/+53 bytes in,
    +11/+19 out), bytes (seed + 37 r + 13 b) % 251."""
    from kvmath import acceptance_rows, strided_rows
    _say("reference acceptance scatter/gather")
    g, lay = _acceptance(goldens)
    geo = lay.kv_pair_copy_geometry(g["layer_index"])
    rb, slots = geo.row_bytes, np.array(g["slots"], np.uint64)
    n = len(slots)
    ks, vs = rb + g["key_stride_extra"], rb + g["value_stride_extra"]
    keys_h, exp_k = acceptance_rows(n, rb, ks, g["key_seed"])
    values_h, exp_v = acceptance_rows(n, rb, vs, g["value_seed"])
    plan = kv.KvPairCopyPlan.new(n, lay.slot_count, geo, ks, vs)
    keys, values = hip.DeviceBuffer.from_array(keys_h), hip.DeviceBuffer.from_array(values_h)
    sl = hip.DeviceBuffer.from_array(slots)
    pool = hip.DeviceBuffer(lay.total_byte_len)
    pool.fill(0)
    k.scatter(plan, keys=keys, values=values, slot_indices=sl, pool=pool)
    got = pool.download()
    touched = np.zeros(lay.total_byte_len, bool)
    for r, slot in enumerate(g["slots"]):
        for t, exp in ((0, exp_k[r]), (1, exp_v[r])):
            s, e = lay.tensor_slot_byte_range(g["layer_index"], t, slot)
            np.testing.assert_array_equal(got[s:e], exp)
            touched[s:e] = True
    assert not got[~touched].any(), "scatter wrote outside the declared slot ranges"
    # the literal byte-per-thread restatement agrees on the whole pool
    want = np.zeros(lay.total_byte_len, np.uint8)
    assert oracle.ref_scatter_kv_pair_bytes(
        keys_h, values_h, slots, want, slot_count=lay.slot_count, page_size=geo.page_size,
        page_stride_bytes=geo.page_stride_bytes, key_in_page_offset=geo.key_in_page_offset,
        value_in_page_offset=geo.value_in_page_offset, row_bytes=rb, key_row_stride_bytes=ks,
        value_row_stride_bytes=vs) == 0
    np.testing.assert_array_equal(got, want)

    gks, gvs = rb + g["gathered_key_stride_extra"], rb + g["gathered_value_stride_extra"]
    gplan = kv.KvPairCopyPlan.new(n, lay.slot_count, geo, gks, gvs)
    gk, gv = hip.DeviceBuffer(gplan.key_rows_required_bytes), hip.DeviceBuffer(gplan.value_rows_required_bytes)
    gk.fill(0)
    gv.fill(0)
    k.gather(gplan, pool=pool, slot_indices=sl, keys=gk, values=gv)
    np.testing.assert_array_equal(strided_rows(gk.download(), n, rb, gks), np.stack(exp_k))
    np.testing.assert_array_equal(strided_rows(gv.download(), n, rb, gvs), np.stack(exp_v))


def test_pair_gather_out_of_range_slot_is_flagged_and_skipped(k):
    _say("pair gather with an out-of-range slot")
    lay = kv.KvPairCopyLayout(2, 64, 0, 16, 8)
    plan = kv.KvPairCopyPlan.new(2, 8, lay, 8, 8)
    pool_h = np.arange(4 * 64, dtype=np.uint8)
    pool = hip.DeviceBuffer.from_array(pool_h)
    sl = hip.DeviceBuffer.from_array(np.array([1, 9], np.uint64))
    keys, values = hip.DeviceBuffer(16), hip.DeviceBuffer(16)
    keys.fill(0xEE)
    values.fill(0xEE)
    with pytest.raises(kv.KvError) as ei:
        k.gather(plan, pool=pool, slot_indices=sl, keys=keys, values=values)
    assert ei.value.variant == "DeviceSlotIndexOutOfRange" and ei.value.fields[0] == 8
    kh, vh = keys.download(), values.download()
    np.testing.assert_array_equal(kh[:8], pool_h[8:16])
    np.testing.assert_array_equal(vh[:8], pool_h[24:32])
    assert (kh[8:] == 0xEE).all() and (vh[8:] == 0xEE).all()
    # the reported error was consumed: check_errors (which asynchronous
    # calls report through) does not see it again
    k.check_errors()
    # the flag was cleared: a valid call afterwards succeeds
    sl.upload(np.array([1, 7], np.uint64))
    k.gather(plan, pool=pool, slot_indices=sl, keys=keys, values=values)


def test_pair_host_checks_reject_before_launch(k):
    _say("pair API host-side range and device checks")
    lay = kv.KvPairCopyLayout(2, 64, 0, 16, 8)
    plan = kv.KvPairCopyPlan.new(2, 8, lay, 8, 8)
    pool = hip.DeviceBuffer(4 * 64)
    sl = hip.DeviceBuffer.from_array(np.array([0, 1], np.uint64))
    keys, values = hip.DeviceBuffer(15), hip.DeviceBuffer(16)
    with pytest.raises(kv.KvError) as ei:
        k.gather(plan, pool=pool, slot_indices=sl, keys=keys, values=values)
    assert ei.value.variant == "AllocationOutOfBounds" and ei.value.name == "keys"
    assert ei.value.fields == (0, 16, 15)
    host = np.zeros(16, np.uint8)
    with pytest.raises(kv.KvError) as ei:
        k.gather(plan, pool=pool, slot_indices=sl, keys=kv.device_buffer(host.ctypes.data, 16),
                 values=values)
    assert ei.value.variant == "DeviceMismatch" and ei.value.name == "keys"


# --- pack / unpack against the oracle ------------------------------------------------------------

def _run_pack_unpack(k, t, layers, seed, fp8_scales=False):
    sh = t.shape
    rb, n, T = sh.row_bytes, t.rows, sh.tensors
    rng = np.random.default_rng(seed)
    src_h = rng.integers(0, 256, t.src.byte_len(sh), dtype=np.uint8)
    dst_h = rng.integers(0, 256, t.dst.byte_len(sh), dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    rows = hip.DeviceBuffer(len(layers) * T * n * rb)
    scales_h = rng.standard_normal(sh.layers * T).astype(np.float32)
    scales = hip.DeviceBuffer.from_array(scales_h)
    out_scales = hip.DeviceBuffer(len(layers) * T * 4)
    dst_scales = hip.DeviceBuffer(sh.layers * T * 4)
    dst_scales.fill(0)
    for i, layer in enumerate(layers):
        sc_src = scales.ptr + layer * T * 4 if fp8_scales else None
        sc_rows = out_scales.ptr + i * T * 4 if fp8_scales else None
        sc_dst = dst_scales.ptr + layer * T * 4 if fp8_scales else None
        base = rows.ptr + i * T * n * rb
        rv = kv.rows_view([base + t_ * n * rb for t_ in range(T)], [n * rb] * T, [rb] * T, sc_rows)
        k.pack_layer(_kpool(src, t.src, sh, layer, sc_src), _db(ss), n, rv)
        k.unpack_layer(rv, n, _kpool(dst, t.dst, sh, layer, sc_dst), _db(ds))
    k.check_errors()
    got_rows, got_dst = rows.download(), dst.download()
    want_rows = np.zeros(len(layers) * T * n * rb, np.uint8)
    want_dst = dst_h.copy()
    for i, layer in enumerate(layers):
        chunk = want_rows[i * T * n * rb:(i + 1) * T * n * rb]
        r0, r1 = chunk[: n * rb], (chunk[n * rb:] if T == 2 else None)
        oracle.pack(_opool(t.src, sh, layer), src_h, t.src_slots, r0, r1, rb, rb, threads=4)
        oracle.unpack(_opool(t.dst, sh, layer), want_dst, t.dst_slots, r0, r1, rb, rb, threads=4)
    np.testing.assert_array_equal(got_rows, want_rows)
    np.testing.assert_array_equal(got_dst, want_dst)
    if fp8_scales:
        sel = np.concatenate([scales_h[l * T:(l + 1) * T] for l in layers]).view(np.uint32)
        np.testing.assert_array_equal(out_scales.download(dtype=np.uint32), sel)
        ds_h = dst_scales.download(dtype=np.uint32)
        for l in layers:
            np.testing.assert_array_equal(ds_h[l * T:(l + 1) * T], scales_h[l * T:(l + 1) * T].view(np.uint32))


def test_c1_full_size_matches_oracle(k):
    """The reference's CPU-runnable configuration, every layer, full size."""
    t = wl.c1()
    _say(f"C1 full size: {t.rows} rows x {t.shape.layers} layers")
    _run_pack_unpack(k, t, range(t.shape.layers), seed=11)


@pytest.mark.parametrize("name,make,max_rows,layers", [
    ("C2", wl.c2, 4096, (0, 13, 31)),
    ("C3-hnd", wl.c3, 9000, (0, 41, 79)),
    ("C4-mla-bf16", lambda: wl.c4(fp8=False), 4096, (0, 30, 60)),
    ("C5-prefix", wl.c5, 6000, (0, 31)),
])
def test_scaled_configs_match_oracle(k, name, make, max_rows, layers):
    t = wl.scaled(make(), max_rows, seed=len(name))
    _say(f"{name}: {t.rows} rows, layers {layers}")
    _run_pack_unpack(k, t, layers, seed=len(name) + 100)


def test_c4_fp8_rows_and_scales_pass_through(k):
    t = wl.scaled(wl.c4(fp8=True), 3000, seed=9)
    _say(f"C4 fp8: {t.rows} rows with per-layer scales")
    _run_pack_unpack(k, t, (0, 1, 60), seed=99, fp8_scales=True)


def test_hnd_with_eight_heads_both_directions(k):
    """C3 has one head, where HND and NHD bytes coincide; eight heads make a
    head/token transpose bug visible. Source HND P=16 -> destination NHD P=64
    and NHD P=1 -> HND P=64."""
    base = wl.scaled(wl.c2(), 2000, seed=3)
    for src_layout, src_p, dst_layout in ((kv.HND, 16, kv.NHD), (kv.NHD, 1, kv.HND)):
        t = wl.scaled(base, 2000, seed=4)
        rows = t.rows
        pages = rows // src_p + 40
        t.src = wl.PoolSpec(src_p, pages, src_layout)
        t.src_slots = np.random.default_rng(5).permutation(pages * src_p)[:rows].astype(np.uint64)
        t.dst = wl.PoolSpec(64, t.dst.page_count, dst_layout)
        _say(f"8-head relayout {src_layout}->{dst_layout}: {rows} rows")
        _run_pack_unpack(k, t, (0, 31), seed=src_p)


@pytest.mark.parametrize("head_major", [True, False])
def test_64_byte_head_chunks(k, head_major):
    """Head chunks of 64 bytes (the hnd64 / nhd64 bench configurations:
    Llama-3.2-1B's 8 KV heads x 64 dims in fp8): P=1 NHD -> P=64 HND, where
    head-major pages are written half a cache line per token, and the same
    into NHD, against the oracle on 3,000 rows of the first and last layers."""
    t = wl.scaled(wl.chunks64(head_major=head_major), 3000, seed=8)
    _say(f"64-byte head chunks, head-major {head_major}: {t.rows} rows")
    _run_pack_unpack(k, t, (0, t.shape.layers - 1), seed=64)


@pytest.mark.parametrize("heads,head_dim,elt", [(8, 8, 2), (4, 32, 1), (8, 32, 2), (2, 16, 4)])
def test_head_chunks_under_a_line_every_direction(k, heads, head_dim, elt):
    """Head chunks of 16, 32 and 64 bytes, where the kernels regroup their
    lanes so that a head-major line's consecutive positions share a wave:
    P16 HND -> P64 NHD and P1 NHD -> P64 HND through pack and unpack, and
    P64 HND -> P32 HND pool -> pool, against the oracle."""
    sh = wl.Shape(3, heads, head_dim, elt, 2)
    base = wl.scaled(wl.c2(), 1500, seed=9)
    base.shape = sh
    _say(f"head chunks of {head_dim * elt} B: {heads} heads, {base.rows} rows")
    for src_layout, src_p, dst_layout, dst_p in ((kv.HND, 16, kv.NHD, 64), (kv.NHD, 1, kv.HND, 64)):
        t = wl.scaled(base, 1500, seed=10)
        t.shape = sh
        pages = t.rows // src_p + 40
        t.src = wl.PoolSpec(src_p, pages, src_layout)
        t.src_slots = np.random.default_rng(11).permutation(pages * src_p)[:t.rows].astype(np.uint64)
        t.dst = wl.PoolSpec(dst_p, t.dst.page_count, dst_layout)
        _run_pack_unpack(k, t, (0, 2), seed=src_p + head_dim)
    t = wl.scaled(base, 1500, seed=12)
    t.shape = sh
    t.src = wl.PoolSpec(64, -(-t.rows // 64) + 8, kv.HND)
    _, _, t.src_slots = wl._page_table_slots(np.random.default_rng(13), t.lengths, np.zeros(len(t.lengths), int),
                                             64, t.src.page_count)
    dst_pages = -(-t.rows // 32) + 8
    t.dst = wl.PoolSpec(32, dst_pages, kv.HND)
    _, _, t.dst_slots = wl._page_table_slots(np.random.default_rng(14), t.lengths, np.zeros(len(t.lengths), int),
                                             32, dst_pages)
    rng = np.random.default_rng(15)
    src_h = rng.integers(0, 256, t.src.byte_len(sh), dtype=np.uint8)
    dst_h = rng.integers(0, 256, t.dst.byte_len(sh), dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    for layer in range(sh.layers):
        k.transfer_layer(_kpool(src, t.src, sh, layer), _db(ss), t.rows, _kpool(dst, t.dst, sh, layer), _db(ds))
        oracle.transfer(_opool(t.src, sh, layer), src_h, t.src_slots, _opool(t.dst, sh, layer), dst_h,
                        t.dst_slots, threads=4)
    k.check_errors()
    np.testing.assert_array_equal(dst.download(), dst_h)


def test_transfer_layer_matches_oracle(k):
    """Pool -> pool in one pass, for co-resident pools (P=1 NHD -> P=64 HND,
    and MLA P=64 -> P=64)."""
    for t in (wl.scaled(wl.c2(), 3000, seed=6), wl.scaled(wl.c4(), 3000, seed=7)):
        if t.shape.tensors == 2:
            t.dst = wl.PoolSpec(64, t.dst.page_count, kv.HND)
        sh = t.shape
        _say(f"transfer_layer {t.name}")
        rng = np.random.default_rng(21)
        src_h = rng.integers(0, 256, t.src.byte_len(sh), dtype=np.uint8)
        dst_h = rng.integers(0, 256, t.dst.byte_len(sh), dtype=np.uint8)
        src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
        ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
        for layer in (0, sh.layers - 1):
            k.transfer_layer(_kpool(src, t.src, sh, layer), _db(ss), t.rows,
                             _kpool(dst, t.dst, sh, layer), _db(ds))
            oracle.transfer(_opool(t.src, sh, layer), src_h, t.src_slots, _opool(t.dst, sh, layer),
                            dst_h, t.dst_slots, threads=4)
        k.check_errors()
        np.testing.assert_array_equal(dst.download(), dst_h)


# --- spans + page table ----------------------------------------------------------------------------

def test_resolve_spans_matches_oracle_and_workload(k):
    t = wl.scaled(wl.c5(), 20000, seed=8)
    _say(f"resolve_spans: {len(t.dst_spans)} spans, {t.rows} rows, prefixes cached")
    spans = hip.DeviceBuffer.from_array(t.dst_spans)
    pt = hip.DeviceBuffer.from_array(t.dst_page_table)
    out = hip.DeviceBuffer(8 * t.rows)
    k.resolve_spans(64, t.dst.page_count, _db(spans), len(t.dst_spans), _db(pt),
                    len(t.dst_page_table), t.rows, _db(out))
    k.check_errors()
    got = out.download(dtype=np.uint64)
    np.testing.assert_array_equal(got, t.dst_slots)
    want, flag = oracle.resolve_slots(_opool(t.dst, t.shape, 0), t.rows,
                                      page_table=t.dst_page_table, spans=t.dst_spans)
    assert flag == 0
    np.testing.assert_array_equal(got, want)


def test_resolve_spans_flags_bad_pages_and_uncovered_rows(k):
    _say("resolve_spans error flags")
    spans_h = np.zeros(2, dtype=kv.SPAN_DTYPE)
    spans_h[0] = (0, 0, 2, 0)
    spans_h[1] = (2, 0, 2, 1)   # rows 2-3 use page_table[1] = 7 (>= 3 pages)
    pt_h = np.array([2, 7], np.int32)
    spans, pt = hip.DeviceBuffer.from_array(spans_h), hip.DeviceBuffer.from_array(pt_h)
    out = hip.DeviceBuffer(8 * 5)   # row 4 is not covered
    k.resolve_spans(4, 3, _db(spans), 2, _db(pt), 2, 5, _db(out))
    with pytest.raises(kv.KvError) as ei:
        k.check_errors()
    assert ei.value.variant == "DevicePageIndexOutOfRange"
    got = out.download(dtype=np.uint64)
    pool = oracle.Pool(4, 64, 3, (0, 32), 16, 2, 1, False)
    want, flag = oracle.resolve_slots(pool, 5, page_table=pt_h, spans=spans_h)
    assert flag == oracle.FLAG_PAGE | oracle.FLAG_SPAN
    np.testing.assert_array_equal(got, want)
    k.check_errors()  # cleared
    # only an uncovered row
    out2 = hip.DeviceBuffer(8 * 3)
    k.resolve_spans(4, 3, _db(spans), 1, _db(pt), 2, 3, _db(out2))
    with pytest.raises(kv.KvError) as ei:
        k.check_errors()
    assert ei.value.variant == "DeviceSpanOutOfRange"


# --- edge cases --------------------------------------------------------------------------------------

def _small_setup(rows, P=4, L=2, H=2, D=8, seed=0):
    shape = wl.Shape(L, H, D, 2, 2)
    rng = np.random.default_rng(seed)
    spec = wl.PoolSpec(P, max(2, -(-rows // P) * 2))
    pool_h = rng.integers(0, 256, spec.byte_len(shape), dtype=np.uint8)
    slots = rng.permutation(spec.page_count * P)[:rows].astype(np.uint64)
    return shape, spec, pool_h, slots


@pytest.mark.parametrize("rows", [1, 7, 8, 63, 64, 65, 513])
def test_ragged_row_counts(k, rows):
    """Row counts around the 8-row thread unroll and the workgroup tile."""
    shape, spec, pool_h, slots = _small_setup(rows, seed=rows)
    rb = shape.row_bytes
    pool, sl = hip.DeviceBuffer.from_array(pool_h), hip.DeviceBuffer.from_array(slots)
    out = hip.DeviceBuffer(2 * rows * rb)
    out.fill(0x5A)
    rv = kv.rows_view([out.ptr, out.ptr + rows * rb], [rows * rb] * 2, [rb, rb])
    k.pack_layer(_kpool(pool, spec, shape, 1), _db(sl), rows, rv)
    k.check_errors()
    want = np.zeros(2 * rows * rb, np.uint8)
    oracle.pack(_opool(spec, shape, 1), pool_h, slots, want[: rows * rb], want[rows * rb:], rb, rb)
    np.testing.assert_array_equal(out.download(), want)


def test_empty_transfer_is_a_noop(k):
    shape, spec, pool_h, slots = _small_setup(4)
    pool, sl = hip.DeviceBuffer.from_array(pool_h), hip.DeviceBuffer.from_array(slots)
    rv = kv.rows_view([pool.ptr, pool.ptr], [0, 0], [shape.row_bytes] * 2)
    k.unpack_layer(rv, 0, _kpool(pool, spec, shape, 0), _db(sl))
    k.pack_layer(_kpool(pool, spec, shape, 0), _db(sl), 0, rv)
    k.check_errors()
    np.testing.assert_array_equal(pool.download(), pool_h)


@pytest.mark.parametrize("extra", [8, 4, 2, 1, 24])
def test_unaligned_row_strides_use_narrower_vectors(k, extra):
    """Row strides of row_bytes + extra force 8/4/2/1-byte accesses."""
    rows = 37
    shape, spec, pool_h, slots = _small_setup(rows, seed=extra)
    rb = shape.row_bytes
    stride = rb + extra
    pool, sl = hip.DeviceBuffer.from_array(pool_h), hip.DeviceBuffer.from_array(slots)
    plane = (rows - 1) * stride + rb
    out = hip.DeviceBuffer(2 * plane + 3)
    out.fill(0x11)
    rv = kv.rows_view([out.ptr, out.ptr + plane + 3], [plane, plane], [stride, stride])
    k.pack_layer(_kpool(pool, spec, shape, 1), _db(sl), rows, rv)
    # and back into a fresh pool
    dst = hip.DeviceBuffer.from_array(np.zeros_like(pool_h))
    k.unpack_layer(rv, rows, _kpool(dst, spec, shape, 1), _db(sl))
    k.check_errors()
    want = np.full(2 * plane + 3, 0x11, np.uint8)
    oracle.pack(_opool(spec, shape, 1), pool_h, slots, want[:plane], want[plane + 3:], stride, stride)
    np.testing.assert_array_equal(out.download(), want)
    want_dst = np.zeros_like(pool_h)
    oracle.unpack(_opool(spec, shape, 1), want_dst, slots, want[:plane], want[plane + 3:], stride, stride)
    np.testing.assert_array_equal(dst.download(), want_dst)


def test_out_of_range_slot_skips_row_and_reports(k):
    rows = 20
    shape, spec, pool_h, slots = _small_setup(rows, seed=3)
    rb = shape.row_bytes
    bad = slots.copy()
    bad[5] = spec.page_count * spec.page_size      # first slot past the pool
    bad[11] = np.uint64(2**63)
    pool, sl = hip.DeviceBuffer.from_array(pool_h), hip.DeviceBuffer.from_array(bad)
    out = hip.DeviceBuffer(2 * rows * rb)
    out.fill(0x77)
    rv = kv.rows_view([out.ptr, out.ptr + rows * rb], [rows * rb] * 2, [rb, rb])
    k.pack_layer(_kpool(pool, spec, shape, 0), _db(sl), rows, rv)
    with pytest.raises(kv.KvError) as ei:
        k.check_errors()
    assert ei.value.variant == "DeviceSlotIndexOutOfRange"
    k.check_errors()  # the word was cleared
    want = np.full(2 * rows * rb, 0x77, np.uint8)
    rs, _ = oracle.resolve_slots(_opool(spec, shape, 0), rows, slots=bad)
    oracle.pack(_opool(spec, shape, 0), pool_h, rs, want[: rows * rb], want[rows * rb:], rb, rb)
    np.testing.assert_array_equal(out.download(), want)


def test_host_validation_errors(k):
    shape, spec, pool_h, slots = _small_setup(8)
    rb = shape.row_bytes
    pool, sl = hip.DeviceBuffer(spec.byte_len(shape) - 1), hip.DeviceBuffer.from_array(slots)
    out = hip.DeviceBuffer(2 * 8 * rb)
    rv = kv.rows_view([out.ptr, out.ptr + 8 * rb], [8 * rb] * 2, [rb, rb])
    with pytest.raises(kv.KvError) as ei:
        k.pack_layer(_kpool(pool, spec, shape, 1), _db(sl), 8, rv)
    assert ei.value.variant == "AllocationOutOfBounds" and ei.value.name == "pool"
    pool = hip.DeviceBuffer(spec.byte_len(shape))
    with pytest.raises(kv.KvError) as ei:
        k.pack_layer(_kpool(pool, spec, shape, 1), _db(sl), 9, rv)
    assert ei.value.variant == "AllocationOutOfBounds" and ei.value.name == "slot_indices"
    rv_small = kv.rows_view([out.ptr, out.ptr + 8 * rb], [8 * rb - 1, 8 * rb], [rb, rb])
    with pytest.raises(kv.KvError) as ei:
        k.pack_layer(_kpool(pool, spec, shape, 1), _db(sl), 8, rv_small)
    assert ei.value.variant == "AllocationOutOfBounds" and ei.value.name == "keys"
    rv_stride = kv.rows_view([out.ptr, out.ptr + 8 * rb], [8 * rb] * 2, [rb - 2, rb])
    with pytest.raises(kv.KvError) as ei:
        k.pack_layer(_kpool(pool, spec, shape, 1), _db(sl), 8, rv_stride)
    assert ei.value.variant == "RowStrideTooSmall"


# --- layer pipeline (pack -> pinned-host hop -> unpack) ----------------------------------------

def _pipeline_case(k, t, staged, seed):
    sh = t.shape
    rb, n, T, L = sh.row_bytes, t.rows, sh.tensors, sh.layers
    rng = np.random.default_rng(seed)
    src_h = rng.integers(0, 256, t.src.byte_len(sh), dtype=np.uint8)
    dst_h = rng.integers(0, 256, t.dst.byte_len(sh), dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    layer_bytes = T * n * rb
    send = [hip.DeviceBuffer(layer_bytes) for _ in range(2)]
    recv = [hip.DeviceBuffer(layer_bytes) for _ in range(2)] if staged else None
    host = [hip.PinnedBuffer(layer_bytes) for _ in range(2)] if staged else None
    pipe = kv.LayerPipeline(k, [_kpool(src, t.src, sh, l) for l in range(L)],
                            [_kpool(dst, t.dst, sh, l) for l in range(L)], _db(ss), _db(ds), n,
                            send, recv, host)
    want = dst_h.copy()
    rows = [np.zeros(n * rb, np.uint8) for _ in range(T)]
    for l in range(L):
        oracle.pack(_opool(t.src, sh, l), src_h, t.src_slots, rows[0], rows[1] if T == 2 else None,
                    rb, rb, threads=4)
        oracle.unpack(_opool(t.dst, sh, l), want, t.dst_slots, rows[0], rows[1] if T == 2 else None,
                      rb, rb, threads=4)
    for run in range(2):
        if run:
            dst.upload(dst_h)
        pipe.run()
        pipe.wait()
        np.testing.assert_array_equal(dst.download(), want)
        times = [pipe.layer_times(l) for l in range(L)]
        assert all(tt[0] > 0 and tt[3] > 0 for tt in times)
        assert all((tt[1] > 0 and tt[2] > 0) == staged for tt in times)
        assert pipe.elapsed_ms() >= max(tt[4] for tt in times) * 0.999
    pipe.close()


def test_staged_pipeline_matches_oracle(k):
    """C5 shape: cached prefixes, pack -> D2H -> pinned host -> H2D -> unpack
    over all 32 layers, run twice (buffer reuse across runs)."""
    t = wl.scaled(wl.c5(), 5000, seed=12)
    _say(f"staged pipeline: {t.rows} rows x {t.shape.layers} layers")
    _pipeline_case(k, t, staged=True, seed=31)


def test_direct_pipeline_matches_oracle(k):
    t = wl.scaled(wl.c3(), 9000, seed=13)
    _say(f"direct pipeline (HND dst): {t.rows} rows x {t.shape.layers} layers")
    _pipeline_case(k, t, staged=False, seed=32)


def test_pipeline_rejects_short_staging_buffers(k):
    t = wl.scaled(wl.c2(), 100, seed=14)
    sh = t.shape
    src, dst = hip.DeviceBuffer(t.src.byte_len(sh)), hip.DeviceBuffer(t.dst.byte_len(sh))
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    lb = 2 * t.rows * sh.row_bytes
    send = [hip.DeviceBuffer(lb), hip.DeviceBuffer(lb)]
    recv = [hip.DeviceBuffer(lb), hip.DeviceBuffer(lb - 16)]
    host = [hip.PinnedBuffer(lb), hip.PinnedBuffer(lb)]
    with pytest.raises(kv.KvError) as ei:
        kv.LayerPipeline(k, [_kpool(src, t.src, sh, l) for l in range(2)],
                         [_kpool(dst, t.dst, sh, l) for l in range(2)], _db(ss), _db(ds), t.rows,
                         send, recv, host)
    assert ei.value.variant == "AllocationOutOfBounds" and ei.value.name == "recv[1]"


# --- multi-layer launches ----------------------------------------------------------------------------

def _multi_layer_case(k, t, seed, fp8_scales=False):
    sh = t.shape
    rb, n, T, L = sh.row_bytes, t.rows, sh.tensors, sh.layers
    rng = np.random.default_rng(seed)
    src_h = rng.integers(0, 256, t.src.byte_len(sh), dtype=np.uint8)
    dst_h = rng.integers(0, 256, t.dst.byte_len(sh), dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    layer_bytes = T * n * rb
    rows = hip.DeviceBuffer(L * layer_bytes)
    scales_h = rng.standard_normal(L * T).astype(np.float32)
    sc_src = hip.DeviceBuffer.from_array(scales_h)
    sc_rows, sc_dst = hip.DeviceBuffer(L * T * 4), hip.DeviceBuffer(L * T * 4)
    rv = kv.rows_view([rows.ptr + i * n * rb for i in range(T)],
                      [L * layer_bytes - i * n * rb for i in range(T)], [rb] * T,
                      sc_rows.ptr if fp8_scales else None)
    sv = _kpool(src, t.src, sh, 0, sc_src.ptr if fp8_scales else None)
    dv = _kpool(dst, t.dst, sh, 0, sc_dst.ptr if fp8_scales else None)
    k.pack_layers(sv, t.src.page_size * T * rb, L, _db(ss), n, rv, layer_bytes)
    k.unpack_layers(rv, layer_bytes, L, n, dv, t.dst.page_size * T * rb, _db(ds))
    k.check_errors()
    want_rows = np.zeros(L * layer_bytes, np.uint8)
    want_dst = dst_h.copy()
    for l in range(L):
        part = want_rows[l * layer_bytes:(l + 1) * layer_bytes]
        r0, r1 = part[: n * rb], (part[n * rb:] if T == 2 else None)
        oracle.pack(_opool(t.src, sh, l), src_h, t.src_slots, r0, r1, rb, rb, threads=4)
        oracle.unpack(_opool(t.dst, sh, l), want_dst, t.dst_slots, r0, r1, rb, rb, threads=4)
    np.testing.assert_array_equal(rows.download(), want_rows)
    np.testing.assert_array_equal(dst.download(), want_dst)
    if fp8_scales:
        np.testing.assert_array_equal(sc_rows.download(dtype=np.uint32), scales_h.view(np.uint32))
        np.testing.assert_array_equal(sc_dst.download(dtype=np.uint32), scales_h.view(np.uint32))


def test_multi_layer_c1_full_size(k):
    """Every layer of C1 in one pack launch and one unpack launch."""
    t = wl.c1()
    _say(f"multi-layer C1: {t.rows} rows x {t.shape.layers} layers per launch")
    _multi_layer_case(k, t, seed=41)


@pytest.mark.parametrize("name,make,max_rows", [
    ("C3-hnd", wl.c3, 3000), ("C4-fp8", lambda: wl.c4(fp8=True), 2000), ("C5", wl.c5, 3000)])
def test_multi_layer_scaled_configs(k, name, make, max_rows):
    t = wl.scaled(make(), max_rows, seed=len(name) + 50)
    _say(f"multi-layer {name}: {t.rows} rows x {t.shape.layers} layers")
    _multi_layer_case(k, t, seed=len(name), fp8_scales=name == "C4-fp8")


def test_multi_layer_validation(k):
    t = wl.scaled(wl.c2(), 100, seed=15)
    sh = t.shape
    rb, n = sh.row_bytes, t.rows
    src, dst = hip.DeviceBuffer(t.src.byte_len(sh)), hip.DeviceBuffer(t.dst.byte_len(sh))
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)
    rows = hip.DeviceBuffer(34 * 2 * n * rb)
    rv = kv.rows_view([rows.ptr, rows.ptr + n * rb], [34 * 2 * n * rb, 34 * 2 * n * rb - n * rb], [rb, rb])
    sv, dv = _kpool(src, t.src, sh, 0), _kpool(dst, t.dst, sh, 0)
    # 33 layers run past the pool's pages (the rows buffer holds 34)
    with pytest.raises(kv.KvError) as ei:
        k.pack_layers(sv, t.src.page_size * 2 * rb, 33, _db(ss), n, rv, 2 * n * rb)
    assert ei.value.variant == "TensorPageRegionOutOfBounds"
    # 35 layers also run past the rows buffer, which is checked first
    with pytest.raises(kv.KvError) as ei:
        k.pack_layers(sv, t.src.page_size * 2 * rb, 35, _db(ss), n, rv, 2 * n * rb)
    assert ei.value.variant == "AllocationOutOfBounds" and ei.value.name == "values"
    # destination rows of consecutive layers would overlap
    with pytest.raises(kv.KvError) as ei:
        k.pack_layers(sv, t.src.page_size * 2 * rb, 4, _db(ss), n, rv, n * rb)
    assert ei.value.variant == "InvalidArgument" and ei.value.name == "rows_layer_stride"
    # destination pool layers would overlap
    with pytest.raises(kv.KvError) as ei:
        k.unpack_layers(rv, 2 * n * rb, 4, n, dv, t.dst.page_size * rb, _db(ds))
    assert ei.value.variant == "InvalidArgument" and ei.value.name == "pool_layer_stride"
    with pytest.raises(kv.KvError) as ei:
        k.unpack_layers(rv, 2 * n * rb, 0, n, dv, t.dst.page_size * 2 * rb, _db(ds))
    assert ei.value.variant == "InvalidArgument" and ei.value.name == "layer_count"


# --- randomized shapes ------------------------------------------------------------------------------

def _random_case(rng):
    T = int(rng.integers(1, 3))
    H = int(rng.choice([1, 2, 3, 4, 8]))
    elt = int(rng.choice([1, 2, 4]))
    D = int(rng.choice([1, 3, 8, 24, 64, 128, 160]))
    L = int(rng.integers(1, 4))
    rb = H * D * elt
    src = wl.PoolSpec(int(rng.choice([1, 2, 16, 64])), 0, int(rng.integers(0, 2)))
    dst = wl.PoolSpec(int(rng.choice([1, 4, 16, 64])), 0, int(rng.integers(0, 2)))
    rows = int(rng.choice([1, 5, 64, 200, 777, 2048]))
    src.page_count = -(-rows // src.page_size) + int(rng.integers(0, 4))
    dst.page_count = -(-rows // dst.page_size) + int(rng.integers(0, 4))
    shape = wl.Shape(L, H, D, elt, T)
    ss = rng.permutation(src.page_count * src.page_size)[:rows].astype(np.uint64)
    ds = rng.permutation(dst.page_count * dst.page_size)[:rows].astype(np.uint64)
    extra = int(rng.choice([0, 0, 16, 1, 2, 4, 8, 48]))
    return shape, src, dst, ss, ds, rows, rb + extra


@pytest.mark.parametrize("seed", range(64))
def test_random_shapes_pack_unpack_transfer(k, seed):
    """Random T, heads, dim, element size, page sizes, NHD/HND on either
    side, row strides and row counts: pack, unpack and pool-to-pool against
    the oracle on the same bytes."""
    rng = np.random.default_rng(1000 + seed)
    sh, sspec, dspec, ss, ds, rows, stride = _random_case(rng)
    rb, T = sh.row_bytes, sh.tensors
    layer = int(rng.integers(0, sh.layers))
    _say(f"random case {seed}: T={T} H={sh.heads} D={sh.head_dim} elt={sh.elt_bytes} rows={rows} "
         f"P {sspec.page_size}{'H' if sspec.head_layout else 'N'}->{dspec.page_size}"
         f"{'H' if dspec.head_layout else 'N'} stride={stride}")
    src_h = rng.integers(0, 256, sspec.byte_len(sh), dtype=np.uint8)
    dst_h = rng.integers(0, 256, dspec.byte_len(sh), dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    sb, dbuf = hip.DeviceBuffer.from_array(ss), hip.DeviceBuffer.from_array(ds)
    plane = (rows - 1) * stride + rb
    rows_buf = hip.DeviceBuffer(T * plane)
    rows_buf.fill(0x3C)
    rv = kv.rows_view([rows_buf.ptr + t_ * plane for t_ in range(T)], [plane] * T, [stride] * T)
    k.pack_layer(_kpool(src, sspec, sh, layer), _db(sb), rows, rv)
    k.unpack_layer(rv, rows, _kpool(dst, dspec, sh, layer), _db(dbuf))
    k.check_errors()
    want_rows = np.full(T * plane, 0x3C, np.uint8)
    r0, r1 = want_rows[:plane], (want_rows[plane:] if T == 2 else None)
    oracle.pack(_opool(sspec, sh, layer), src_h, ss, r0, r1, stride, stride)
    want_dst = dst_h.copy()
    oracle.unpack(_opool(dspec, sh, layer), want_dst, ds, r0, r1, stride, stride)
    np.testing.assert_array_equal(rows_buf.download(), want_rows)
    np.testing.assert_array_equal(dst.download(), want_dst)
    # pool -> pool of another layer, into a fresh destination
    layer2 = int(rng.integers(0, sh.layers))
    dst2_h = rng.integers(0, 256, dspec.byte_len(sh), dtype=np.uint8)
    dst2 = hip.DeviceBuffer.from_array(dst2_h)
    k.transfer_layer(_kpool(src, sspec, sh, layer2), _db(sb), rows, _kpool(dst2, dspec, sh, layer2),
                     _db(dbuf))
    k.check_errors()
    oracle.transfer(_opool(sspec, sh, layer2), src_h, ss, _opool(dspec, sh, layer2), dst2_h, ds)
    np.testing.assert_array_equal(dst2.download(), dst2_h)


# --- page-request execution (the reference's page-for-page PD transfer) ------------------------------

@pytest.mark.parametrize("page_bytes,pages", [(3072, 40), (100, 17), (8 << 20, 6)])
def test_execute_page_requests_local(k, page_bytes, pages):
    """build_page_requests -> device copies: target page page_offset + i of the
    destination segment receives source page page_indices[i]."""
    rng = np.random.default_rng(page_bytes)
    src_pages, page_size = pages * 3, 4
    src_h = rng.integers(0, 256, src_pages * page_bytes, dtype=np.uint8)
    src = hip.DeviceBuffer.from_array(src_h)
    target_base_offset, token_offset = 2 * page_bytes, 8
    dst_bytes = target_base_offset + (token_offset // page_size + pages) * page_bytes
    dst_h = rng.integers(0, 256, dst_bytes, dtype=np.uint8)
    dst = hip.DeviceBuffer.from_array(dst_h)
    page_indices = rng.permutation(src_pages)[:pages]
    reqs = kv.build_page_requests(src.ptr, page_bytes, target_base_offset, token_offset,
                                  pages * page_size - 1, page_size, page_indices)
    rq = hip.DeviceBuffer.from_array(reqs)
    k.execute_page_requests(_db(rq), len(reqs), page_bytes, _db(src), _db(dst))
    k.check_errors()
    want = dst_h.copy()
    for i, p in enumerate(page_indices):
        t0 = target_base_offset + (token_offset // page_size + i) * page_bytes
        want[t0:t0 + page_bytes] = src_h[p * page_bytes:(p + 1) * page_bytes]
    np.testing.assert_array_equal(dst.download(), want)


def test_execute_remote_page_requests_split_over_pointers(k):
    """The decode side advertises 4 per-split regions (dst_kv_ptrs) of one
    device buffer; each source page lands split by split at its index."""
    rng = np.random.default_rng(7)
    PB, J, pages, slots = 8192, 4, 33, 50
    item = PB // J
    src_h = rng.integers(0, 256, 80 * PB, dtype=np.uint8)
    src = hip.DeviceBuffer.from_array(src_h)
    dst = hip.DeviceBuffer(J * slots * item)
    dst.fill(0)
    ptrs = [dst.ptr + j * slots * item for j in range(J)]
    page_indices = rng.permutation(80)[:pages]
    dst_idx = rng.permutation(slots)[:pages].astype(np.int32)
    reqs = kv.build_remote_page_requests(src.ptr, PB, pages, 1, page_indices, ptrs, dst_idx, item)
    rq = hip.DeviceBuffer.from_array(reqs)
    k.execute_page_requests(_db(rq), len(reqs), item, _db(src), _db(dst), offsets_are_addresses=True)
    k.check_errors()
    got = dst.download().reshape(J, slots, item)
    for i, p in enumerate(page_indices):
        np.testing.assert_array_equal(got[:, dst_idx[i], :], src_h[p * PB:(p + 1) * PB].reshape(J, item))


def test_execute_page_requests_skips_and_reports_out_of_region(k):
    rng = np.random.default_rng(9)
    PB = 4096
    src_h = rng.integers(0, 256, 8 * PB, dtype=np.uint8)
    src = hip.DeviceBuffer.from_array(src_h)
    dst = hip.DeviceBuffer(8 * PB)
    dst.fill(0)
    reqs = kv.build_page_requests(src.ptr, PB, 0, 0, 3, 1, [1, 7, 2])
    reqs[1]["source"] = src.ptr + 8 * PB          # past the source region
    bad_target = reqs.copy()
    bad_target[0]["target_offset"] = 8 * PB - 16  # runs past the target region
    rq = hip.DeviceBuffer.from_array(reqs)
    k.execute_page_requests(_db(rq), 3, PB, _db(src), _db(dst))
    with pytest.raises(kv.KvError) as ei:
        k.check_errors()
    assert ei.value.variant == "DeviceRequestOutOfRange"
    got = dst.download()
    np.testing.assert_array_equal(got[:PB], src_h[PB:2 * PB])
    assert not got[PB:2 * PB].any()
    np.testing.assert_array_equal(got[2 * PB:3 * PB], src_h[2 * PB:3 * PB])
    rq.upload(bad_target)
    k.execute_page_requests(_db(rq), 3, PB, _db(src), _db(dst))
    with pytest.raises(kv.KvError):
        k.check_errors()
    # a request longer than the launch's max_length covers is skipped, not cut
    big_h = rng.integers(0, 256, 1 << 17, dtype=np.uint8)
    big, big_dst = hip.DeviceBuffer.from_array(big_h), hip.DeviceBuffer(1 << 17)
    big_dst.fill(0)
    one = hip.DeviceBuffer.from_array(kv.build_page_requests(big.ptr, 1 << 17, 0, 0, 1, 1, [0]))
    k.execute_page_requests(_db(one), 1, 1 << 16, _db(big), _db(big_dst))
    with pytest.raises(kv.KvError):
        k.check_errors()
    assert not big_dst.download().any()
    k.execute_page_requests(_db(one), 1, 1 << 17, _db(big), _db(big_dst))
    k.check_errors()
    np.testing.assert_array_equal(big_dst.download(), big_h)
