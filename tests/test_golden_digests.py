"""Frozen results: the pack and unpack of small seeded transfers
(tests/golden/pool_cases.py: C1's geometry, eight heads into head-major
pages, DeepSeek-V3's 1,152/1,024-byte pair, 649-byte packed-MLA rows,
576-byte fp8 latent rows, 64-byte head chunks) hash to the SHA-256 digests
committed in tests/golden/pool_digests.json, which make_pool_digests.py
computed by numpy indexing of the layout views.

On the CPU the inputs, the numpy route and the C oracle are checked against
the digests; on the GPU (marked gpu) the product's kernels, through the C
ABI, are.
"""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import pool_cases  # noqa: E402

DIGESTS = json.load(open(os.path.join(HERE, "golden", "pool_digests.json")))
NAMES = [c.name for c in pool_cases.CASES]


def _sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _case(name):
    return next(c for c in pool_cases.CASES if c.name == name)


def test_every_case_has_digests():
    assert sorted(NAMES) == sorted(k for k in DIGESTS if not k.startswith("_"))


@pytest.mark.parametrize("name", NAMES)
def test_inputs_match_digests(name):
    c, d = _case(name), DIGESTS[name]
    assert _sha(c.src_pool()) == d["src_pool"] and _sha(c.dst_pool()) == d["dst_pool_before"]
    assert _sha(c.src_slots()) == d["src_slots"] and _sha(c.dst_slots()) == d["dst_slots"]
    assert len(set(c.src_slots().tolist())) == c.tokens and len(set(c.dst_slots().tolist())) == c.tokens


@pytest.mark.parametrize("name", NAMES)
def test_numpy_route_matches_digests(name):
    rows, dst = pool_cases.numpy_pack_unpack(_case(name))
    assert _sha(rows) == DIGESTS[name]["rows"] and _sha(dst) == DIGESTS[name]["dst_pool_after"]
    assert DIGESTS[name]["dst_pool_after"] != DIGESTS[name]["dst_pool_before"]


def _opool(c, side, layer):
    w = c.widths
    return oracle.Pool(side.page_size, side.page_stride(c), side.page_count, tuple(side.tensor_offsets(c, layer)),
                       w[0], len(w), c.heads, side.hnd, w[1] if len(w) == 2 and w[1] != w[0] else 0)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_digests(name):
    c = _case(name)
    src, dst = c.src_pool(), c.dst_pool()
    ss, ds = c.src_slots(), c.dst_slots()
    rows = np.zeros(c.rows_bytes(), dtype=np.uint8)
    n = c.tokens
    for layer in range(c.layers):
        planes = [rows[c.plane_offset(layer, t): c.plane_offset(layer, t) + n * w] for t, w in enumerate(c.widths)]
        second = planes[1] if len(planes) == 2 else None
        stride1 = c.widths[1] if len(planes) == 2 else 0
        oracle.pack(_opool(c, c.src, layer), src, ss, planes[0], second, c.widths[0], stride1)
        oracle.unpack(_opool(c, c.dst, layer), dst, ds, planes[0], second, c.widths[0], stride1)
    assert _sha(rows) == DIGESTS[name]["rows"] and _sha(dst) == DIGESTS[name]["dst_pool_after"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_gpu_matches_digests(name):
    import sgl_rocm_kv as kv
    from sgl_rocm_kv import hip
    if hip.device_count() == 0:
        pytest.fail("no GPU visible: the gpu tests need an MI355X")
    c = _case(name)
    print(f"[gpu] golden digests: {name} ({c.layers} layers x {c.tokens} tokens, widths {c.widths})", flush=True)
    n, w = c.tokens, c.widths
    with kv.RocmKvPairCopyKernels(0) as k:
        src = hip.DeviceBuffer.from_array(c.src_pool())
        dst = hip.DeviceBuffer.from_array(c.dst_pool())
        ss = hip.DeviceBuffer.from_array(c.src_slots())
        ds = hip.DeviceBuffer.from_array(c.dst_slots())
        rows = hip.DeviceBuffer(c.rows_bytes())

        def view(buf, side, layer):
            return kv.pool_view(buf.ptr, buf.nbytes, page_size=side.page_size,
                                page_stride_bytes=side.page_stride(c), page_count=side.page_count,
                                tensor_offset=side.tensor_offsets(c, layer), row_bytes=w[0],
                                tensor_count=len(w), heads=c.heads, head_layout=kv.HND if side.hnd else kv.NHD,
                                value_row_bytes=w[1] if len(w) == 2 and w[1] != w[0] else 0)

        for layer in range(c.layers):
            rv = kv.rows_view([rows.ptr + c.plane_offset(layer, t) for t in range(len(w))],
                              [n * x for x in w], list(w))
            k.pack_layer(view(src, c.src, layer), kv.device_buffer(ss.ptr, ss.nbytes), n, rv)
            k.unpack_layer(rv, n, view(dst, c.dst, layer), kv.device_buffer(ds.ptr, ds.nbytes))
        k.check_errors()
        got_rows, got_dst = rows.download(), dst.download()
    assert _sha(got_rows) == DIGESTS[name]["rows"]
    assert _sha(got_dst) == DIGESTS[name]["dst_pool_after"]
