"""KvCacheModelLayout and paged_kv_cache_layout_for_model on the CPU: the
product's mirror (sgl_kv_model_layout_*, sgl_kv_paged_layout_for_model)
against the reference's own test values and error messages, and the pair
layout it produces against the oracle's independently written byte ranges
on random shapes. No kernel is launched here.
"""
import numpy as np
import pytest

import oracle
import sgl_rocm_kv as kv


def test_asymmetric_tensor_pair_golden(goldens):
    """crates/sglang-srt/tests/kv_cache.rs:180-217."""
    g = goldens["model_layout"]["asymmetric_pair"]
    m = kv.KvCacheModelLayout.tensor_pair(*g["args"])
    assert m.elements_per_token() == g["elements_per_token"]
    assert m.token_size_bytes("bf16") == g["token_size_bytes_bf16"]
    assert m.tensor_pair_size_bytes("bf16") == g["tensor_pair_size_bytes_bf16"]
    assert m.kv_tensors_per_token == 2 and m.kv_heads == 1 and m.head_dim == 5
    # The runtime layout of that test: page 4, 2 pages (slot capacity 8).
    lay = kv.PagedKvCacheLayout.for_model(m, "bf16", 4, 8)
    pair = goldens["asymmetric_pair"]
    assert lay.total_byte_len == pair["total_byte_len"]
    for r in pair["ranges"]:
        assert lay.tensor_token_byte_range(*r["args"]) == tuple(r["range"]), r
    rt = lay.runtime
    assert (rt.page_size, rt.bytes_per_token, rt.page_size_bytes) == (4, 32, 128)


def test_deepseek_v3_pair_golden(goldens):
    """crates/sglang-srt/src/model_registry.rs:538-553, 777-783."""
    g = goldens["model_layout"]["deepseek_v3_test_config"]
    m = kv.KvCacheModelLayout.tensor_pair(*g["args"])
    assert m.num_layers == 2
    assert m.tensor_pair_size_bytes("float32") == g["tensor_pair_size_bytes_float32"]


def test_deepseek_v3_full_size_pair_pool():
    """The pool the DeepSeek-V3 adapter allocates (models/deepseek.rs:360-369:
    tensor_pair(61, 1, 512 + 64, 1, 512)) in bf16 at page 64: keys 1,152 and
    values 1,024 bytes per token per layer; a two-tensor view carries both
    widths."""
    m = kv.KvCacheModelLayout.tensor_pair(61, 1, 576, 1, 512)
    assert m.token_size_bytes("bf16") == 61 * (1152 + 1024)
    lay = kv.PagedKvCacheLayout.for_model(m, "bf16", 64, 64 * 10)
    assert lay.tensor_token_bytes(0) == 1152 and lay.tensor_token_bytes(1) == 1024
    v = lay.pool_view(0x1000, lay.total_byte_len, 60)
    assert v.tensor_count == 2 and v.row_bytes == 1152 and v.value_row_bytes == 1024
    assert v.tensor_row_bytes(1) == 1024
    assert list(v.tensor_offset) == [60 * 64 * 2176, 60 * 64 * 2176 + 64 * 1152]
    # kv_pair_copy_geometry keeps the reference's rejection of unequal widths
    with pytest.raises(kv.KvError) as ei:
        lay.kv_pair_copy_geometry(0)
    assert ei.value.variant == "UnevenKvPairCopy" and list(ei.value.fields[:2]) == [1152, 1024]


def test_packed_mla_golden(goldens):
    """packed_mla (kv_cache.rs:201-224) as build_mla_moe_definition uses it
    (models/deepseek.rs:1035-1037): one byte row per token per layer whatever
    the dtype."""
    g = goldens["model_layout"]["packed_mla_deepseek"]
    m = kv.KvCacheModelLayout.packed_mla(*g["args"])
    assert m.bytes_per_token_per_layer == g["bytes_per_token_per_layer"]
    assert (m.kv_heads, m.head_dim, m.kv_tensors_per_token) == (1, 649, 1)
    assert m.elements_per_token() is None and m.tensor_pair_size_bytes("fp8_e4m3") is None
    for dtype in ("bf16", "fp8_e4m3", "fp4_e2m1", "float32"):
        assert m.token_size_bytes(dtype) == 61 * 649
    lay = kv.PagedKvCacheLayout.for_model(m, "fp8_e4m3", 64, 64 * 4)
    assert lay.bytes_per_token_per_tensor == 649 and lay.bytes_per_layer_page == 64 * 649
    v = lay.pool_view(0x1000, lay.total_byte_len, 7)
    assert v.tensor_count == 1 and v.row_bytes == 649 and v.value_row_bytes == 0
    assert v.tensor_offset[0] == 7 * 64 * 649


def test_model_layout_errors(goldens):
    e = goldens["model_layout"]["errors"]
    g = e["packed_mla_nope_not_multiple_of_64"]
    with pytest.raises(kv.KvError) as ei:
        kv.KvCacheModelLayout.packed_mla(*g["args"])
    assert ei.value.variant == g["variant"] and list(ei.value.fields[:1]) == g["fields"]
    assert str(ei.value.message) == g["message"]
    g = e["tensor_pair_zero_width"]
    with pytest.raises(kv.KvError) as ei:
        kv.KvCacheModelLayout.tensor_pair(*g["args"])
    assert ei.value.variant == g["variant"] and str(ei.value.message) == g["message"]
    with pytest.raises(kv.KvError) as ei:
        kv.KvCacheModelLayout.multi_tensor(2, 1, 8, 2).token_size_bytes("fp4_e2m1")
    assert ei.value.variant == "DtypeRequiresModelMetadata"
    assert ei.value.fields[0] == kv.DTYPES["fp4_e2m1"]
    assert str(ei.value.message) == e["fp4_needs_metadata"]["message"]
    with pytest.raises(kv.KvError) as ei:
        kv.KvCacheModelLayout.tensor_pair(1, 2**63, 4, 1, 1)
    assert ei.value.variant == "SizeOverflow"
    with pytest.raises(kv.KvError) as ei:
        kv.KvCacheModelLayout.packed_mla(1, 64, 2**63)
    assert ei.value.variant == "SizeOverflow"
    # elements_per_token is None on overflow, and token_size_bytes reports it
    big = kv.KvCacheModelLayout.multi_tensor(2**40, 2**20, 2**10, 2)
    assert big.elements_per_token() is None
    with pytest.raises(kv.KvError) as ei:
        big.token_size_bytes("bf16")
    assert ei.value.variant == "SizeOverflow"


@pytest.mark.parametrize("cap,ps,key", [(0, 4, "zero_capacity"), (8, 0, "zero_page_size"),
                                        (10, 4, "unaligned")])
def test_cache_config_is_validated(goldens, cap, ps, key):
    """validate_cache_config (backend_model.rs:457-475)."""
    m = kv.KvCacheModelLayout.multi_tensor(2, 1, 8, 2)
    with pytest.raises(kv.KvError) as ei:
        kv.PagedKvCacheLayout.for_model(m, "bf16", ps, cap)
    assert ei.value.variant == "MissingCapabilities"
    assert goldens["model_layout"]["cache_config_messages"][key] in str(ei.value.message)


def test_multi_tensor_matches_the_runtime_for_model_helper():
    """for_model on multi_tensor gives the Uniform layout the runtime helper
    builds (the GQA models, e.g. models/qwen.rs:234-239)."""
    m = kv.KvCacheModelLayout.multi_tensor(32, 8, 128, 2)
    a = kv.PagedKvCacheLayout.for_model(m, "bf16", 64, 64 * 16)
    b = kv.PagedKvCacheLayout.new(kv.KvCacheRuntimeLayout.for_model("bf16", 64, 32, 8, 128), 16)
    assert a.runtime == b.runtime and a.total_byte_len == b.total_byte_len
    assert a.bytes_per_token_per_tensor == 2048


def test_pair_layouts_agree_with_the_oracle_on_random_shapes():
    """The product's tensor-pair byte ranges (every layer, tensor, token of
    random unequal-width pairs) equal the oracle's pair ranges, which the
    asymmetric goldens and a numpy view pin independently
    (tests/test_oracle.py)."""
    rng = np.random.default_rng(3)
    for _ in range(25):
        L, P, pages = int(rng.integers(1, 5)), int(rng.choice([1, 2, 16, 64])), int(rng.integers(1, 4))
        kd, vd = int(rng.integers(1, 700)), int(rng.integers(1, 600))
        dtype = str(rng.choice(["bf16", "fp8_e4m3", "float32"]))
        m = kv.KvCacheModelLayout.tensor_pair(L, 1, kd, 1, vd)
        lay = kv.PagedKvCacheLayout.for_model(m, dtype, P, P * pages)
        kb, vb = m.tensor_pair_size_bytes(dtype)
        rt = lay.runtime
        olay = oracle.layout(P, L, 2, rt.bytes_per_token, rt.page_size_bytes, pages)
        for _ in range(20):
            page, layer = int(rng.integers(0, pages)), int(rng.integers(0, L))
            t, tok = int(rng.integers(0, 2)), int(rng.integers(0, P))
            rc, want = oracle.pair_tensor_token_byte_range(olay, kb, vb, page, layer, t, tok)
            assert rc == 0 and lay.tensor_token_byte_range(page, layer, t, tok) == want
            slot = page * P + tok
            assert lay.tensor_slot_byte_range(layer, t, slot) == want
        # and the layer view the copies take
        v = lay.pool_view(0x1000, lay.total_byte_len, L - 1)
        rc, k0 = oracle.pair_tensor_token_byte_range(olay, kb, vb, 0, L - 1, 0, 0)
        rc2, v0 = oracle.pair_tensor_token_byte_range(olay, kb, vb, 0, L - 1, 1, 0)
        assert (v.tensor_offset[0], v.tensor_offset[1]) == (k0[0], v0[0])
        assert (v.row_bytes, v.tensor_row_bytes(1)) == (kb, vb)
