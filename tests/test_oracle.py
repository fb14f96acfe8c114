"""Pins the CPU oracle (oracle/kv_oracle.c) before anything is compared with it.

Every oracle function is checked against at least one of: a golden value
from the reference's own tests, a numpy reshape view of the pool (an
independent derivation of the layout), a brute-force literal restatement, or
a library routine. No test here retypes the oracle's own formula.
"""
import numpy as np
import pytest

import oracle
from kvmath import (acceptance_rows, pool_view, rows_from_view, slots_from_page_table,
                    strided_rows, write_rows_to_view)

STATUS = {
    "PageOutOfRange": 26, "LayerOutOfRange": 27, "TensorOutOfRange": 28,
    "TokenOutOfRange": 29, "SlotOutOfRange": 30,
}


def _lay(rt, page_count):
    return oracle.layout(rt["page_size"], rt["num_layers"], rt["kv_tensors_per_token"],
                         rt["bytes_per_token"], rt["page_size_bytes"], page_count)


# --- layout goldens (crates/sglang-srt/tests/kv_cache.rs) -------------------------------

def test_layout_goldens(goldens):
    g = goldens["kv_cache_layout"]
    lay = _lay(g["runtime"], g["page_count"])
    assert oracle.tensor_token_byte_range(lay, 1, 1, 1, 3) == (0, tuple(g["tensor_token_byte_range_1_1_1_3"]))
    assert oracle.tensor_slot_byte_range(lay, 1, 1, 7) == (0, tuple(g["tensor_slot_byte_range_1_1_7"]))
    for e in g["errors"]:
        if e["call"] == "page_byte_range":
            continue
        fn = getattr(oracle, e["call"])
        rc, _ = fn(lay, *e["args"])
        assert rc == STATUS[e["variant"]], e


def test_cuda_backend_slot_location_golden(goldens):
    # slot_location(layer 1, tensor 1, slot 63) == offset 522,240, len 2,048
    # (crates/sglang-srt/tests/cuda_backend.rs:284-286).
    g = goldens["cuda_backend_slot_location"]
    lay = _lay(g["runtime"], g["page_count"])
    rc, (s, e) = oracle.tensor_slot_byte_range(lay, 1, 1, 63)
    want = g["slot_location_layer_1_tensor_1_slot_63"]
    assert rc == 0 and s == want["byte_offset"] and e - s == want["byte_len"]


def test_asymmetric_pair_goldens(goldens):
    g = goldens["asymmetric_pair"]
    lay = _lay(g["runtime"], g["page_count"])
    for r in g["ranges"]:
        rc, rng = oracle.pair_tensor_token_byte_range(lay, g["key_token_bytes"], g["value_token_bytes"], *r["args"])
        assert rc == 0 and rng == tuple(r["range"]), r


@pytest.mark.parametrize("P,L,T,rb,pages", [(4, 2, 2, 32, 3), (16, 3, 2, 64, 5), (1, 4, 1, 48, 7), (64, 2, 2, 16, 2)])
def test_layout_matches_reshape_view(P, L, T, rb, pages):
    """Every (slot, layer, tensor) range starts where the numpy view
    [page][layer][tensor][token][row] puts that row."""
    lay = oracle.layout(P, L, T, L * T * rb, P * L * T * rb, pages)
    total = pages * P * L * T * rb
    index = np.arange(total, dtype=np.int64)
    view = index.reshape(pages, L, T, P, rb)
    for slot in range(pages * P):
        for layer in range(L):
            for t in range(T):
                rc, (s, e) = oracle.tensor_slot_byte_range(lay, layer, t, slot)
                assert rc == 0
                assert s == view[slot // P, layer, t, slot % P, 0] and e - s == rb


# --- literal reference kernels vs the reference acceptance test -----------------------

def _acceptance_setup(goldens):
    g = goldens["scatter_gather_acceptance"]
    rt = goldens["cuda_backend_slot_location"]["runtime"]
    lay = _lay(rt, g["page_count"])
    rb = rt["kv_heads"] * rt["head_dim"] * 2
    per_layer_page = rt["page_size"] * rt["bytes_per_token"] // rt["num_layers"]
    layer = g["layer_index"]
    geom = dict(page_size=rt["page_size"], page_stride_bytes=rt["page_size_bytes"],
                key_in_page_offset=layer * per_layer_page,
                value_in_page_offset=layer * per_layer_page + rt["page_size"] * rb, row_bytes=rb)
    return g, rt, lay, rb, geom


def test_reference_scatter_gather_acceptance(goldens):
    """cuda_kv_kernels_scatter_and_gather_batched_physical_slots
    (crates/sglang-srt/tests/cuda_backend.rs:497-637), run on the literal
    byte-per-thread restatement."""
    g, rt, lay, rb, geom = _acceptance_setup(goldens)
    slots = np.array(g["slots"], dtype=np.uint64)
    n = len(slots)
    ks, vs = rb + g["key_stride_extra"], rb + g["value_stride_extra"]
    keys, exp_k = acceptance_rows(n, rb, ks, g["key_seed"])
    values, exp_v = acceptance_rows(n, rb, vs, g["value_seed"])
    pool = np.zeros(g["page_count"] * rt["page_size_bytes"], dtype=np.uint8)
    slot_count = g["page_count"] * rt["page_size"]
    flag = oracle.ref_scatter_kv_pair_bytes(keys, values, slots, pool, slot_count=slot_count,
                                            key_row_stride_bytes=ks, value_row_stride_bytes=vs, **geom)
    assert flag == 0
    touched = np.zeros_like(pool, dtype=bool)
    for r, slot in enumerate(g["slots"]):
        for t, exp in ((0, exp_k[r]), (1, exp_v[r])):
            rc, (s, e) = oracle.tensor_slot_byte_range(lay, g["layer_index"], t, slot)
            assert rc == 0
            np.testing.assert_array_equal(pool[s:e], exp)
            touched[s:e] = True
    assert not pool[~touched].any(), "scatter wrote outside the declared slot ranges"

    gks, gvs = rb + g["gathered_key_stride_extra"], rb + g["gathered_value_stride_extra"]
    gk = np.zeros((n - 1) * gks + rb, dtype=np.uint8)
    gv = np.zeros((n - 1) * gvs + rb, dtype=np.uint8)
    flag = oracle.ref_gather_kv_pair_bytes(pool, slots, gk, gv, slot_count=slot_count,
                                           key_row_stride_bytes=gks, value_row_stride_bytes=gvs, **geom)
    assert flag == 0
    np.testing.assert_array_equal(strided_rows(gk, n, rb, gks), np.stack(exp_k))
    np.testing.assert_array_equal(strided_rows(gv, n, rb, gvs), np.stack(exp_v))


def test_reference_gather_flags_out_of_range_slot():
    pool = np.arange(4 * 64, dtype=np.uint8)
    keys = np.full(2 * 8, 0xEE, dtype=np.uint8)
    values = np.full(2 * 8, 0xEE, dtype=np.uint8)
    flag = oracle.ref_gather_kv_pair_bytes(
        pool, np.array([1, 9], dtype=np.uint64), keys, values, slot_count=8, page_size=2,
        page_stride_bytes=64, key_in_page_offset=0, value_in_page_offset=16, row_bytes=8,
        key_row_stride_bytes=8, value_row_stride_bytes=8)
    assert flag == 1
    assert (keys[8:] == 0xEE).all() and (values[8:] == 0xEE).all(), "bad row must be skipped"
    np.testing.assert_array_equal(keys[:8], pool[8:16])
    np.testing.assert_array_equal(values[:8], pool[24:32])


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_reference_gather_matches_numpy_view(seed):
    rng = np.random.default_rng(seed)
    P, L, H, D, pages = 16, 3, 2, 8, 6
    rb = H * D * 2
    pool = rng.integers(0, 256, pages * P * L * 2 * rb, dtype=np.uint8)
    view = pool_view(pool, pages, L, 2, P, rb)
    n, layer = 23, 2
    slots = rng.permutation(pages * P)[:n].astype(np.uint64)
    keys = np.zeros(n * rb, dtype=np.uint8)
    values = np.zeros(n * rb, dtype=np.uint8)
    flag = oracle.ref_gather_kv_pair_bytes(
        pool, slots, keys, values, slot_count=pages * P, page_size=P,
        page_stride_bytes=P * L * 2 * rb, key_in_page_offset=layer * P * 2 * rb,
        value_in_page_offset=layer * P * 2 * rb + P * rb, row_bytes=rb,
        key_row_stride_bytes=rb, value_row_stride_bytes=rb)
    assert flag == 0
    np.testing.assert_array_equal(keys.reshape(n, rb), rows_from_view(view, slots, layer, 0, P, False))
    np.testing.assert_array_equal(values.reshape(n, rb), rows_from_view(view, slots, layer, 1, P, False))


# --- generalised pack / unpack ------------------------------------------------------------

def _pool(P, L, T, rb, H, hnd, pages, layer):
    return oracle.Pool(page_size=P, page_stride=P * L * T * rb, page_count=pages,
                       tensor_offset=tuple(layer * P * T * rb + t * P * rb for t in range(T)),
                       row_bytes=rb, tensors=T, heads=H, hnd=hnd)


@pytest.mark.parametrize("P,L,T,H,D,hnd", [(1, 3, 2, 2, 8, False), (16, 2, 2, 4, 8, False),
                                             (8, 2, 2, 4, 8, True), (4, 2, 1, 1, 24, False),
                                             (64, 1, 2, 8, 4, True)])
def test_pack_matches_numpy_view(P, L, T, H, D, hnd):
    rng = np.random.default_rng(P * 31 + H)
    rb, pages, layer = H * D * 2, 5, L - 1
    pool = rng.integers(0, 256, pages * P * L * T * rb, dtype=np.uint8)
    view = pool_view(pool, pages, L, T, P, rb, H, hnd)
    n = min(37, pages * P)
    slots = rng.permutation(pages * P)[:n].astype(np.uint64)
    rows = [np.zeros((n, rb), dtype=np.uint8) for _ in range(2)]
    p = _pool(P, L, T, rb, H, hnd, pages, layer)
    oracle.pack(p, pool, slots, rows[0], rows[1] if T == 2 else None, rb, rb)
    for t in range(T):
        np.testing.assert_array_equal(rows[t], rows_from_view(view, slots, layer, t, P, hnd))


@pytest.mark.parametrize("threads", [1, 3])
def test_pack_agrees_with_literal_reference_on_nhd_pairs(threads):
    rng = np.random.default_rng(7)
    P, L, rb, pages, layer = 16, 2, 64, 4, 1
    pool = rng.integers(0, 256, pages * P * L * 2 * rb, dtype=np.uint8)
    slots = rng.permutation(pages * P)[:29].astype(np.uint64)
    n = len(slots)
    k1, v1 = np.zeros(n * rb, np.uint8), np.zeros(n * rb, np.uint8)
    oracle.ref_gather_kv_pair_bytes(pool, slots, k1, v1, slot_count=pages * P, page_size=P,
                                    page_stride_bytes=P * L * 2 * rb,
                                    key_in_page_offset=layer * P * 2 * rb,
                                    value_in_page_offset=layer * P * 2 * rb + P * rb,
                                    row_bytes=rb, key_row_stride_bytes=rb, value_row_stride_bytes=rb)
    k2, v2 = np.zeros(n * rb, np.uint8), np.zeros(n * rb, np.uint8)
    oracle.pack(_pool(P, L, 2, rb, 1, False, pages, layer), pool, slots, k2, v2, rb, rb, threads)
    np.testing.assert_array_equal(k1, k2)
    np.testing.assert_array_equal(v1, v2)


@pytest.mark.parametrize("hnd", [False, True])
def test_unpack_matches_numpy_view_and_touches_only_its_rows(hnd):
    rng = np.random.default_rng(11)
    P, L, T, H, D, pages, layer = 8, 3, 2, 4, 4, 6, 1
    rb = H * D * 2
    pool = np.zeros(pages * P * L * T * rb, dtype=np.uint8)
    n = 19
    slots = rng.permutation(pages * P)[:n].astype(np.uint64)
    rows = [rng.integers(0, 256, (n, rb), dtype=np.uint8) for _ in range(T)]
    oracle.unpack(_pool(P, L, T, rb, H, hnd, pages, layer), pool, slots, rows[0], rows[1], rb, rb)
    expect = np.zeros_like(pool)
    ev = pool_view(expect, pages, L, T, P, rb, H, hnd)
    for t in range(T):
        write_rows_to_view(ev, slots, layer, t, P, hnd, rows[t])
    np.testing.assert_array_equal(pool, expect)


def test_transfer_equals_pack_then_unpack_across_layouts():
    """Pool-to-pool with P 1 NHD -> P 8 HND equals unpack(pack(.))."""
    rng = np.random.default_rng(5)
    L, T, H, D, layer = 2, 2, 4, 8, 1
    rb = H * D * 2
    sp = _pool(1, L, T, rb, H, False, 128, layer)
    dp = _pool(8, L, T, rb, H, True, 20, layer)
    src = rng.integers(0, 256, 128 * L * T * rb, dtype=np.uint8)
    n = 50
    s_slots = rng.permutation(128)[:n].astype(np.uint64)
    d_slots = rng.permutation(160)[:n].astype(np.uint64)
    a = np.zeros(20 * 8 * L * T * rb, np.uint8)
    oracle.transfer(sp, src, s_slots, dp, a, d_slots)
    k, v = np.zeros((n, rb), np.uint8), np.zeros((n, rb), np.uint8)
    oracle.pack(sp, src, s_slots, k, v, rb, rb)
    b = np.zeros_like(a)
    oracle.unpack(dp, b, d_slots, k, v, rb, rb)
    np.testing.assert_array_equal(a, b)
    # and the destination view holds the source rows
    sv = pool_view(src, 128, L, T, 1, rb, H, False)
    dv = pool_view(a, 20, L, T, 8, rb, H, True)
    for t in range(T):
        np.testing.assert_array_equal(rows_from_view(dv, d_slots, layer, t, 8, True),
                                      rows_from_view(sv, s_slots, layer, t, 1, False))


def _spans(rows_per_req, offsets, page_starts):
    spans = np.zeros(len(rows_per_req), dtype=oracle.SPAN_DTYPE)
    start = 0
    for i, (n, off, ps) in enumerate(zip(rows_per_req, offsets, page_starts)):
        spans[i] = (start, off, n, ps)
        start += n
    return spans


def test_resolve_slots_from_page_table_matches_token_walk():
    rng = np.random.default_rng(3)
    P, pages = 4, 40
    lens = [5, 9, 1, 12]
    offsets = [0, 4, 8, 0]  # page-aligned prefixes already cached on the decode side
    need = [-(-(o + n) // P) for o, n in zip(offsets, lens)]
    perm = rng.permutation(pages).astype(np.int32)
    page_starts = np.concatenate([[0], np.cumsum(need)[:-1]]).astype(int)
    pt = perm[: sum(need)]
    spans = _spans(lens, offsets, page_starts)
    pool = _pool(P, 1, 2, 16, 1, False, pages, 0)
    got, flag = oracle.resolve_slots(pool, sum(lens), page_table=pt, spans=spans)
    assert flag == 0
    np.testing.assert_array_equal(got.astype(np.int64), slots_from_page_table(pt, spans, P))


def test_resolve_slots_flags():
    pool = _pool(4, 1, 2, 16, 1, False, 3, 0)
    got, flag = oracle.resolve_slots(pool, 3, slots=np.array([0, 12, 11]))
    assert flag == oracle.FLAG_SLOT and got[1] == oracle.INVALID_SLOT and got[2] == 11
    spans = _spans([2, 2], [0, 0], [0, 1])
    got, flag = oracle.resolve_slots(pool, 5, page_table=np.array([2, 7], np.int32), spans=spans)
    # rows 2-3 use page 7 (>= 3 pages) -> PAGE; row 4 is not covered -> SPAN
    assert flag == oracle.FLAG_PAGE | oracle.FLAG_SPAN
    assert list(got[:2]) == [8, 9] and all(g == oracle.INVALID_SLOT for g in got[2:])
    got, flag = oracle.resolve_slots(pool, 2, page_table=np.array([-1], np.int32), spans=_spans([2], [0], [0]))
    assert flag == oracle.FLAG_PAGE


# --- transfer plan pages (crates/sglang-srt/src/transfer.rs:679-720) --------------------

def test_transfer_page_indices(goldens):
    g = goldens["transfer_plan"]
    # page_size 1: every slot is its own page (from_prefill_worker_batch uses page size 1).
    rc, pages = oracle.transfer_page_indices(g["span_token_offset"], [20, 21], 1)
    assert rc == 0 and pages == [20, 21] and len(pages) == g["span_cache_pages"]
    assert oracle.transfer_page_indices(0, [8, 9, 10, 11, 4, 5], 4) == (0, [2, 1])
    assert oracle.transfer_page_indices(0, [], 4) == (0, [])
    assert oracle.transfer_page_indices(2, [8, 9], 4)[0] == 43   # UnalignedTokenOffset
    assert oracle.transfer_page_indices(0, [9, 10], 4)[0] == 44  # UnalignedCacheSlot
    assert oracle.transfer_page_indices(0, [8, 10], 4)[0] == 45  # NonContiguousCacheSlots


def test_f32_to_bf16_matches_torch_round_to_nearest_even():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32),
                        np.array([0.0, -0.0, 1.0, -2.5, 3.0e38, -3.0e38, 1e-40, 65504.0,
                                  1.00390625, 1.01171875, np.inf, -np.inf], dtype=np.float32)])
    got = oracle.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
