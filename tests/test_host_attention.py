"""CPU tests of the paged-attention plan (sgl_kv_attention_plan_new /
_for_layer) against the reference's own plan tests
(crates/sglang-kernel/src/cuda_attention.rs:898-1019 and
crates/sglang-srt/tests/cuda_attention.rs:70-168), transcribed into
tests/golden/reference_goldens.json, plus the oracle's attention
restatement pinned against torch's scaled_dot_product_attention."""
import ctypes
import math

import numpy as np
import pytest

import oracle
import sgl_rocm_kv as kv
from kvmath import pool_view, rows_from_view


def _config(base, patch):
    c = dict(base)
    c.update(patch)
    if c["scale"] == "1/sqrt(8)":
        c["scale"] = 1.0 / math.sqrt(8.0)
    lay = c.pop("layout")
    return dict(c, page_size=lay[0], page_stride_bytes=lay[1], key_in_page_offset=lay[2],
                value_in_page_offset=lay[3], key_row_bytes=lay[4], value_row_bytes=lay[5])


def test_plan_goldens(goldens):
    g = goldens["paged_attention_plan"]
    plan = kv.PagedAttentionPlan.new(**_config(g["base_config"], g["gqa"]["patch"]))
    assert (plan.query_count, plan.request_count, plan.sequence_slot_count, plan.slot_count) == (3, 2, 6, 12)
    assert (plan.query_head_count, plan.kv_head_count, plan.query_key_head_dim, plan.value_head_dim) == (4, 2, 8, 8)
    assert plan.layout == tuple(g["base_config"]["layout"])
    for k in ("query_required_bytes", "output_required_bytes", "pool_required_bytes"):
        assert getattr(plan, k) == g["gqa"][k], k
    mla = kv.PagedAttentionPlan.new(**_config(g["base_config"], g["mla_unequal"]["patch"]))
    assert mla.query_required_bytes == g["mla_unequal"]["query_required_bytes"]
    assert mla.output_required_bytes == g["mla_unequal"]["output_required_bytes"]
    assert (mla.key_row_bytes, mla.value_row_bytes) == (24, 16)


def test_plan_errors(goldens):
    g = goldens["paged_attention_plan"]
    for e in g["errors"]:
        with pytest.raises(kv.KvError) as ei:
            kv.PagedAttentionPlan.new(**_config(g["base_config"], e["patch"]))
        assert ei.value.variant == e["variant"], e
        if "name" in e:
            assert ei.value.name == e["name"]
        assert list(ei.value.fields[:len(e["fields"])]) == e["fields"], e


def test_plan_region_errors_keep_the_reference_fields(goldens):
    base = goldens["paged_attention_plan"]["base_config"]
    with pytest.raises(kv.KvError) as ei:   # value region [384, 512+) past the stride
        kv.PagedAttentionPlan.new(**_config(base, {"layout": [4, 512, 256, 400, 32, 32]}))
    assert ei.value.variant == "TensorPageRegionOutOfBounds" and ei.value.name == "value"
    assert ei.value.fields == (400, 128, 512)
    with pytest.raises(kv.KvError) as ei:   # four fields: offsets and both page sizes
        kv.PagedAttentionPlan.new(**_config(base, {"layout": [4, 512, 256, 300, 32, 32]}))
    assert ei.value.variant == "TensorPageRegionsOverlap"
    assert ei.value.fields == (256, 300, 128, 128)
    with pytest.raises(kv.KvError) as ei:
        kv.PagedAttentionPlan.new(**_config(base, {"scale": float("nan")}))
    assert ei.value.variant == "InvalidScale"


def test_plan_flags(goldens):
    """The plan flags (no counterpart in the reference): 0 is the default
    (hi + lo weights everywhere), ATTN_EXACT_WEIGHTS names it and
    ATTN_FAST_WEIGHTS asks the latent body for one bf16 per weight; both
    constructors carry them, plan_new refuses unknown bits and the pair."""
    g = goldens["paged_attention_plan"]
    cfg = _config(g["base_config"], g["gqa"]["patch"])
    assert kv.PagedAttentionPlan.new(**cfg).flags == 0
    plan = kv.PagedAttentionPlan.new(**cfg, exact_weights=True)
    assert plan.flags == kv.ATTN_EXACT_WEIGHTS == 1
    assert kv.PagedAttentionPlan.new(**cfg, fast_weights=True).flags == kv.ATTN_FAST_WEIGHTS == 2
    f = g["from_layout"]
    lay = kv.PagedKvCacheLayout.new(_runtime(f["runtime"]), f["page_count"])
    assert kv.PagedAttentionPlan.for_layer(lay, 1, 5, 2, 5, 4, 0.5, exact_weights=True).flags == 1
    assert kv.PagedAttentionPlan.for_layer(lay, 1, 5, 2, 5, 4, 0.5, fast_weights=True).flags == 2
    for bad in (4, 0x80000000, 3, 7):
        plan._c.config.flags = bad
        out = type(plan._c)()
        with pytest.raises(kv.KvError) as ei:
            kv._call(kv.lib().sgl_kv_attention_plan_new, ctypes.byref(plan._c.config), ctypes.byref(out))
        assert ei.value.name == "flags" and ei.value.fields[:2] == (bad, 3)


def _runtime(rt, dtype=None):
    return kv.KvCacheRuntimeLayout(dtype or rt["dtype"], rt["page_size"], rt["num_layers"], rt["kv_heads"],
                                   rt["head_dim"], rt["kv_tensors_per_token"], rt["bytes_per_token"],
                                   rt["page_size_bytes"])


def test_plan_from_pool_layout(goldens):
    g = goldens["paged_attention_plan"]
    f = g["from_layout"]
    lay = kv.PagedKvCacheLayout.new(_runtime(f["runtime"]), f["page_count"])
    plan = kv.PagedAttentionPlan.for_layer(lay, f["layer"], f["query_count"], f["request_count"],
                                           f["sequence_slot_count"], f["query_head_count"],
                                           1.0 / math.sqrt(8.0))
    for k, v in f["want"].items():
        assert getattr(plan, k) == v, k
    # Key/value offsets of layer 1 are the layout's tensor_token_byte_range.
    assert plan.key_in_page_offset == lay.tensor_token_byte_range(0, 1, 0, 0)[0] == 256
    assert plan.value_in_page_offset == lay.tensor_token_byte_range(0, 1, 1, 0)[0] == 384
    a = g["from_layout_asymmetric"]
    pair = kv.PagedKvCacheLayout.new_with_tensor_pair(_runtime(a["runtime"]), 2, *a["pair"])
    plan = kv.PagedAttentionPlan.for_layer(pair, a["layer"], 5, 2, 5, a["query_head_count"], 1.0)
    assert (plan.query_key_head_dim, plan.value_head_dim) == (8, 4)
    fp8 = kv.PagedKvCacheLayout.new(_runtime(f["runtime"], "fp8_e4m3"), 2)
    with pytest.raises(kv.KvError) as ei:
        kv.PagedAttentionPlan.for_layer(fp8, 0, 5, 2, 5, 4, 1.0)
    assert ei.value.variant == "UnsupportedKvDtype"
    assert list(ei.value.fields[:2]) == g["from_layout_fp8"]["fields"]


# --- the oracle's attention restatement, pinned by a library routine --------------------------

def _sdpa_reference(pool, P, L, H, D, layer, hnd, pages, queries_f, metadata, scale):
    """Independent path: gather rows through the reshape view of the pool
    (page -> layer -> tensor -> token order) and run torch's
    scaled_dot_product_attention in float64 with GQA expanded."""
    torch = pytest.importorskip("torch")
    view = pool_view(pool, pages, L, 2, P, H * D * 2, heads=H, hnd=hnd)
    qri, qsl, rso, slots = metadata
    nq, qh, _ = queries_f.shape
    out = np.zeros((nq, qh, D))
    for q in range(nq):
        r = qri[q]
        sl = np.asarray(slots[rso[r]:rso[r] + qsl[q]], np.int64)
        k = oracle.bf16_to_f32(rows_from_view(view, sl, layer, 0, P, hnd).view(np.uint16)).reshape(-1, H, D)
        v = oracle.bf16_to_f32(rows_from_view(view, sl, layer, 1, P, hnd).view(np.uint16)).reshape(-1, H, D)
        kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2).repeat_interleave(qh // H, 0)
        vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2).repeat_interleave(qh // H, 0)
        qt = torch.from_numpy(queries_f[q].astype(np.float64))[:, None, :]
        o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=scale)
        out[q] = o[:, 0, :].numpy()
    return out


@pytest.mark.parametrize("hnd", [False, True])
def test_oracle_attention_matches_torch_sdpa(hnd):
    rng = np.random.default_rng(3 + hnd)
    P, L, H, D, pages, qh, layer = 4, 3, 2, 16, 12, 8, 1
    page_bytes = P * L * 2 * H * D * 2
    pool = oracle.f32_to_bf16(rng.standard_normal(pages * page_bytes // 2).astype(np.float32)).view(np.uint8)
    lens = [5, 1, 13]
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.permutation(pages * P)[:int(rso[-1])].astype(np.uint64)
    qri = np.array([0, 0, 1, 2, 2], np.uint32)
    qsl = np.array([5, 3, 1, 13, 7], np.uint64)
    queries = oracle.f32_to_bf16(rng.standard_normal((5, qh, D)).astype(np.float32))
    scale = 1.0 / math.sqrt(D)
    key_off = layer * (P * 2 * H * D * 2)
    got, flags = oracle.paged_attention(pool, queries, qri, qsl, rso, slots, page_size=P,
                                        page_stride=page_bytes, key_offset=key_off,
                                        value_offset=key_off + P * H * D * 2, kv_heads=H, dk=D, dv=D,
                                        scale=scale, slot_count=pages * P, hnd=hnd)
    assert flags == 0
    want = _sdpa_reference(pool, P, L, H, D, layer, hnd, pages, oracle.bf16_to_f32(queries),
                           (qri, qsl, rso, slots), scale)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_oracle_attention_pair_layout_matches_torch_sdpa():
    """Unequal key and value widths in a tensor-pair layout, the MLA form
    (576/512 for DeepSeek-V3, 24/16 here): rows gathered through the
    layout's tensor_slot_byte_range (pinned by the reference's layout
    goldens), attention by torch's scaled_dot_product_attention in float64
    with every query head on the one KV head."""
    torch = pytest.importorskip("torch")
    P, L, dk, dv, pages, qh, layer = 4, 2, 24, 16, 6, 8, 1
    kb, vb = dk * 2, dv * 2
    rt = kv.KvCacheRuntimeLayout("bf16", P, L, 1, dk, 2, L * (kb + vb), L * (kb + vb) * P)
    lay = kv.PagedKvCacheLayout.new_with_tensor_pair(rt, pages, kb, vb)
    rng = np.random.default_rng(17)
    pool = oracle.f32_to_bf16(rng.standard_normal(lay.total_byte_len // 2).astype(np.float32)).view(np.uint8)
    lens = [7, 1, 11]
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.permutation(lay.slot_count)[:int(rso[-1])].astype(np.uint64)
    qri, qsl = np.array([0, 1, 2, 2], np.uint32), np.array([7, 1, 11, 4], np.uint64)
    queries = oracle.f32_to_bf16(rng.standard_normal((4, qh, dk)).astype(np.float32))
    scale = 0.3
    plan = kv.PagedAttentionPlan.for_layer(lay, layer, 4, 3, len(slots), qh, scale)
    got, flags = oracle.paged_attention(pool, queries, qri, qsl, rso, slots, page_size=P,
                                        page_stride=plan.page_stride_bytes, key_offset=plan.key_in_page_offset,
                                        value_offset=plan.value_in_page_offset, kv_heads=1, dk=dk, dv=dv,
                                        scale=scale, slot_count=lay.slot_count)
    assert flags == 0

    def rows(sl, tensor):
        out = []
        for s_ in sl:
            a, b = lay.tensor_slot_byte_range(layer, tensor, int(s_))
            out.append(oracle.bf16_to_f32(pool[a:b].view(np.uint16)))
        return np.stack(out).astype(np.float64)

    qf = oracle.bf16_to_f32(queries).astype(np.float64)
    for q in range(4):
        sl = slots[rso[qri[q]]:rso[qri[q]] + qsl[q]]
        kt = torch.from_numpy(rows(sl, 0))[None].expand(qh, -1, -1)
        vt = torch.from_numpy(rows(sl, 1))[None].expand(qh, -1, -1)
        o = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(qf[q])[:, None, :], kt, vt,
                                                             scale=scale)
        np.testing.assert_allclose(got[q], o[:, 0, :].numpy(), rtol=1e-12, atol=1e-12)


def test_oracle_attention_closed_forms_and_flags():
    """One attended token returns its value row exactly; equal keys return
    the mean of the values; bad metadata sets the reference's flag bits."""
    P, H, D, pages = 2, 1, 8, 4
    page_bytes = P * 2 * H * D * 2
    rng = np.random.default_rng(9)
    pool = oracle.f32_to_bf16(rng.standard_normal(pages * page_bytes // 2).astype(np.float32)).view(np.uint8)
    pool16 = pool.view(np.uint16)
    # Equal keys for slots 0..3: copy slot 0's key row into the others.
    key0 = pool16[0:D].copy()
    for s in range(1, 4):
        base = (s // P) * page_bytes // 2 + (s % P) * D
        pool16[base:base + D] = key0
    q = oracle.f32_to_bf16(rng.standard_normal((2, 1, D)).astype(np.float32))
    args = dict(page_size=P, page_stride=page_bytes, key_offset=0, value_offset=P * D * 2, kv_heads=1,
                dk=D, dv=D, scale=0.5, slot_count=pages * P)
    out, flags = oracle.paged_attention(pool, q, [0, 0], [1, 4], [0, 4], [2, 1, 0, 3], **args)
    vrow = lambda s: oracle.bf16_to_f32(pool16[(s // P) * page_bytes // 2 + P * D + (s % P) * D:][:D])
    np.testing.assert_array_equal(out[0, 0], vrow(2))
    np.testing.assert_allclose(out[1, 0], np.mean([vrow(s) for s in range(4)], axis=0), rtol=1e-12)
    assert flags == 0
    # sum_i w_i |v_i| (the error model's weight term): |v| of the one
    # token, the mean of |v| under equal keys; never below |out|.
    out2, flags, absw = oracle.paged_attention(pool, q, [0, 0], [1, 4], [0, 4], [2, 1, 0, 3], with_abs=True,
                                               **args)
    np.testing.assert_array_equal(out2, out)
    np.testing.assert_array_equal(absw[0, 0], np.abs(vrow(2)))
    np.testing.assert_allclose(absw[1, 0], np.mean([np.abs(vrow(s)) for s in range(4)], axis=0), rtol=1e-12)
    assert flags == 0 and (absw >= np.abs(out) - 1e-12).all()
    _, flags = oracle.paged_attention(pool, q, [1, 0], [1, 1], [0, 4], [0, 1, 2, 3], **args)
    assert flags == oracle.FLAG_ATTN_REQUEST
    _, flags = oracle.paged_attention(pool, q, [0, 0], [0, 5], [0, 4], [0, 1, 2, 3], **args)
    assert flags == oracle.FLAG_ATTN_SEQUENCE
    _, flags = oracle.paged_attention(pool, q, [0, 0], [2, 1], [0, 4], [0, 8, 2, 3], **args)
    assert flags == oracle.FLAG_ATTN_SLOT
