"""The product library on the CPU: it loads, exports every function the
C-ABI header declares, and its host mirror of the reference's layout and
plan arithmetic (group 1 of include/sgl_rocm_kv.h) returns the reference's
own golden values and error variants. No kernel is launched here.
"""
import os
import re

import numpy as np
import pytest

import sgl_rocm_kv as kv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = []
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"^\s*[A-Za-z_][\w \*]*?\b(sgl_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_function():
    import ctypes
    names = _declared_functions()
    assert len(names) >= 20, names
    handle = ctypes.CDLL(kv.LIB_PATH)
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, f"declared in include/ but not exported: {missing}"
    # and the binding knows every one of them
    assert sorted(kv.exported_names()) == names


def test_code_object_is_built_for_gfx950():
    with open(kv.CODE_OBJECT_PATH, "rb") as f:
        head = f.read(64)
    assert head[:4] == b"\x7fELF"
    assert int.from_bytes(head[18:20], "little") == 224  # EM_AMDGPU
    # e_flags: EF_AMDGPU_MACH in the low byte; gfx950 = 0x4f
    assert int.from_bytes(head[48:52], "little") & 0xFF == 0x4F


def test_code_object_kernels_spill_nothing():
    """Every kernel of the code object keeps its state in registers and LDS:
    no private (scratch) segment and no VGPR or SGPR spills, read from the
    code object's metadata notes (llvm-readelf --notes, from the ROCm
    toolchain)."""
    import re
    import shutil
    import subprocess
    readelf = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "llvm-readelf")
    if not os.path.exists(readelf):
        readelf = shutil.which("llvm-readelf")
    if not readelf:
        pytest.skip("llvm-readelf is not available to read the code object's notes")
    notes = subprocess.run([readelf, "--notes", kv.CODE_OBJECT_PATH], capture_output=True, text=True,
                           check=True).stdout
    kernels = re.split(r"\n\s+- \.agpr_count:", notes)[1:]
    assert len(kernels) >= 40, len(kernels)
    bad = []
    for k in kernels:
        name = re.search(r"\.name:\s+(\S+)", k).group(1)
        fields = {f: int(re.search(rf"\.{f}:\s+(\d+)", k).group(1))
                  for f in ("private_segment_fixed_size", "vgpr_spill_count", "sgpr_spill_count")}
        if any(fields.values()):
            bad.append((name, fields))
    assert not bad, bad


def _runtime(d, **patch):
    r = dict(d)
    r.update(patch)
    return kv.KvCacheRuntimeLayout(r["dtype"], r["page_size"], r["num_layers"], r["kv_heads"],
                                   r["head_dim"], r["kv_tensors_per_token"], r["bytes_per_token"],
                                   r["page_size_bytes"])


def test_paged_layout_goldens(goldens):
    g = goldens["kv_cache_layout"]
    lay = kv.PagedKvCacheLayout.new(_runtime(g["runtime"]), g["page_count"])
    assert lay.bytes_per_token_per_layer == g["bytes_per_token_per_layer"]
    assert lay.bytes_per_token_per_tensor == g["bytes_per_token_per_tensor"]
    assert lay.bytes_per_layer_page == g["bytes_per_layer_page"]
    assert lay.bytes_per_tensor_page == g["bytes_per_tensor_page"]
    assert lay.total_byte_len == g["total_byte_len"]
    assert lay.slot_count == g["slot_count"]
    assert lay.page_byte_range(1) == tuple(g["page_byte_range_1"])
    assert lay.tensor_token_byte_range(1, 1, 1, 3) == tuple(g["tensor_token_byte_range_1_1_1_3"])
    assert lay.tensor_slot_byte_range(1, 1, 7) == tuple(g["tensor_slot_byte_range_1_1_7"])
    for e in g["errors"]:
        with pytest.raises(kv.KvError) as ei:
            getattr(lay, e["call"])(*e["args"])
        assert ei.value.variant == e["variant"] and list(ei.value.fields[:2]) == e["fields"], e
    geo = lay.kv_pair_copy_geometry(1)
    want = g["kv_pair_copy_geometry_layer_1"]
    assert (geo.page_size, geo.page_stride_bytes, geo.key_in_page_offset,
            geo.value_in_page_offset, geo.row_bytes) == (
        want["page_size"], want["page_stride_bytes"], want["key_offset_bytes"],
        want["value_offset_bytes"], want["token_bytes"])
    lay.validate_slot_indices(g["validate_slot_indices_ok"])
    bad = g["validate_slot_indices_bad"]
    with pytest.raises(kv.KvError) as ei:
        lay.validate_slot_indices(bad["slots"])
    assert ei.value.variant == bad["variant"] and list(ei.value.fields) == bad["fields"]
    with pytest.raises(kv.KvError) as ei:
        lay.validate_slot_indices([])
    assert ei.value.variant == "EmptySlotMap"


def test_paged_layout_runtime_errors(goldens):
    g = goldens["kv_cache_layout"]
    for e in g["runtime_errors"]:
        with pytest.raises(kv.KvError) as ei:
            kv.PagedKvCacheLayout.new(_runtime(g["runtime"], **e["patch"]), e["page_count"])
        assert ei.value.variant == e["variant"] and list(ei.value.fields[:2]) == e["fields"], e
    with pytest.raises(kv.KvError) as ei:
        kv.PagedKvCacheLayout.new(_runtime(g["runtime"]), 0)
    assert ei.value.variant == "ZeroPageCount"
    with pytest.raises(kv.KvError) as ei:
        kv.PagedKvCacheLayout.new(_runtime(g["runtime"], head_dim=0), 1)
    assert ei.value.variant == "ZeroLayoutField" and ei.value.name == "head_dim"


def test_tensor_pair_layout_goldens(goldens):
    g = goldens["asymmetric_pair"]
    lay = kv.PagedKvCacheLayout.new_with_tensor_pair(_runtime(g["runtime"]), g["page_count"],
                                                     g["key_token_bytes"], g["value_token_bytes"])
    assert lay.total_byte_len == g["total_byte_len"]
    assert lay.bytes_per_token_per_tensor is None and lay.bytes_per_tensor_page is None
    for r in g["ranges"]:
        assert lay.tensor_token_byte_range(*r["args"]) == tuple(r["range"]), r
    with pytest.raises(kv.KvError) as ei:
        lay.kv_pair_copy_geometry(0)
    want = g["kv_pair_copy_geometry_layer_0"]
    assert ei.value.variant == want["variant"] and list(ei.value.fields[:2]) == want["fields"]
    base = goldens[g["pair_errors"][0]["base"]]["runtime"]
    for e in g["pair_errors"]:
        with pytest.raises(kv.KvError) as ei:
            kv.PagedKvCacheLayout.new_with_tensor_pair(_runtime(base, **e["patch"]), 1, e["key"],
                                                       e["value"])
        n = len(e["fields"])
        assert ei.value.variant == e["variant"] and list(ei.value.fields[:n]) == e["fields"], e


def test_cuda_backend_slot_location_golden(goldens):
    g = goldens["cuda_backend_slot_location"]
    lay = kv.PagedKvCacheLayout.new(_runtime(g["runtime"]), g["page_count"])
    s, e = lay.tensor_slot_byte_range(1, 1, 63)
    want = g["slot_location_layer_1_tensor_1_slot_63"]
    assert (s, e - s) == (want["byte_offset"], want["byte_len"])
    assert lay.total_byte_len == g["pool_byte_len"]


def test_layout_agrees_with_the_oracle_on_random_shapes():
    """The product's byte ranges equal the (independently pinned) oracle's."""
    import oracle
    rng = np.random.default_rng(0)
    for _ in range(20):
        P, L, T = int(rng.choice([1, 4, 16, 64])), int(rng.integers(1, 5)), int(rng.integers(1, 3))
        H, D, pages = int(rng.integers(1, 5)), int(rng.choice([8, 64, 128])), int(rng.integers(1, 6))
        bpt = L * T * H * D * 2
        rt = kv.KvCacheRuntimeLayout("bf16", P, L, H, D, T, bpt, P * bpt)
        lay = kv.PagedKvCacheLayout.new(rt, pages)
        olay = oracle.layout(P, L, T, bpt, P * bpt, pages)
        for _ in range(10):
            slot, layer, t = int(rng.integers(0, pages * P)), int(rng.integers(0, L)), int(rng.integers(0, T))
            rc, rngo = oracle.tensor_slot_byte_range(olay, layer, t, slot)
            assert rc == 0 and lay.tensor_slot_byte_range(layer, t, slot) == rngo


def test_pair_layout_agrees_with_the_oracle_on_random_pair_shapes():
    """Tensor-pair pools with unequal key and value widths (the MLA form,
    kv_cache.rs:436-823 with key/value token bytes): every byte range the
    product computes, and its pool view's per-tensor row widths, equal the
    oracle's pair arithmetic (pinned by the asymmetric-pair goldens)."""
    import oracle
    rng = np.random.default_rng(7)
    for _ in range(30):
        P, L, pages = int(rng.choice([1, 2, 16, 64])), int(rng.integers(1, 6)), int(rng.integers(1, 5))
        kb = 2 * int(rng.integers(1, 700))
        vb = 2 * int(rng.integers(1, 700))
        if kb == vb:
            vb += 2
        bpt = L * (kb + vb)
        rt = kv.KvCacheRuntimeLayout("bf16", P, L, 1, kb // 2, 2, bpt, P * bpt)
        lay = kv.PagedKvCacheLayout.new_with_tensor_pair(rt, pages, kb, vb)
        olay = oracle.layout(P, L, 2, bpt, P * bpt, pages)
        assert lay.total_byte_len == P * bpt * pages
        for _ in range(12):
            slot, layer, t = int(rng.integers(0, pages * P)), int(rng.integers(0, L)), int(rng.integers(0, 2))
            rc, want = oracle.pair_tensor_token_byte_range(olay, kb, vb, slot // P, layer, t, slot % P)
            assert rc == 0 and lay.tensor_slot_byte_range(layer, t, slot) == want, (P, L, kb, vb, slot, layer, t)
        layer = int(rng.integers(0, L))
        view = lay.pool_view(0x10000, lay.total_byte_len, layer, kv.NHD, 1)
        assert view.tensor_row_bytes(0) == kb and view.tensor_row_bytes(1) == vb
        for t in range(2):
            rc, (s, _) = oracle.pair_tensor_token_byte_range(olay, kb, vb, 0, layer, t, 0)
            assert rc == 0 and view.tensor_offset[t] == s


def test_pair_copy_plan_goldens(goldens):
    g = goldens["pair_copy_plan"]
    lay = kv.KvPairCopyLayout(**g["layout"])
    plan = kv.KvPairCopyPlan.new(3, 12, lay, 40, 48)
    want = g["new_3_12_40_48"]
    assert (plan.key_rows_required_bytes, plan.value_rows_required_bytes,
            plan.slot_indices_required_bytes, plan.pool_required_bytes) == (
        want["key_rows_required_bytes"], want["value_rows_required_bytes"],
        want["slot_indices_required_bytes"], want["pool_required_bytes"])
    assert plan.layout == lay and plan.row_count == 3 and plan.slot_count == 12
    umax = 2**64 - 1
    for e in g["errors"]:
        args = [umax if a == "usize::MAX" else a for a in e["args"]]
        lay_args = [umax if a == "usize::MAX" else a for a in args[2]]
        with pytest.raises(kv.KvError) as ei:
            kv.KvPairCopyPlan.new(args[0], args[1], kv.KvPairCopyLayout(*lay_args), args[3], args[4])
        assert ei.value.variant == e["variant"], e
        if "name" in e:
            assert ei.value.name == e["name"]
        n = len(e["fields"])
        assert list(ei.value.fields[:n]) == e["fields"], e


def test_transfer_page_indices(goldens):
    g = goldens["transfer_plan"]
    assert kv.transfer_page_indices(0, g["span_token_offset"], [20, 21], 1) == [20, 21]
    assert kv.transfer_page_indices(0, 0, [8, 9, 10, 11, 4, 5], 4) == [2, 1]
    assert kv.transfer_page_indices(0, 0, [], 4) == []
    for args, variant in [((7, 2, [8, 9], 4), "UnalignedTokenOffset"),
                          ((7, 0, [9, 10], 4), "UnalignedCacheSlot"),
                          ((7, 0, [8, 10], 4), "NonContiguousCacheSlots"),
                          ((7, 0, [8], 0), "ZeroPageSize")]:
        with pytest.raises(kv.KvError) as ei:
            kv.transfer_page_indices(*args)
        assert ei.value.variant == variant
    with pytest.raises(kv.KvError) as ei:
        kv.transfer_page_indices(7, 0, [8, 10], 4)
    assert ei.value.fields == (7, 9, 10)


def test_transfer_page_indices_agrees_with_oracle():
    import oracle
    rng = np.random.default_rng(1)
    for _ in range(50):
        P = int(rng.choice([1, 2, 4, 16]))
        pages = rng.permutation(40)[: int(rng.integers(0, 6))]
        slots = np.concatenate([p * P + np.arange(P) for p in pages]).astype(np.uint64) if len(pages) else np.zeros(0, np.uint64)
        if len(slots) and rng.random() < 0.3:
            slots = slots[: int(rng.integers(1, len(slots) + 1))]
        if len(slots) and rng.random() < 0.3:
            slots[int(rng.integers(0, len(slots)))] += 1
        rc, want = oracle.transfer_page_indices(0, slots, P)
        if rc == 0:
            assert kv.transfer_page_indices(0, 0, slots, P) == want
        else:
            with pytest.raises(kv.KvError) as ei:
                kv.transfer_page_indices(0, 0, slots, P)
            assert ei.value.code == rc


def test_pool_view_for_layer():
    rt = kv.KvCacheRuntimeLayout.for_model("bf16", 64, 32, 8, 128)
    lay = kv.PagedKvCacheLayout.new(rt, 4)
    v = lay.pool_view(0x1000, lay.total_byte_len, 3, kv.HND, 8)
    assert v.page_size == 64 and v.page_stride_bytes == 64 * 32 * 2 * 2048
    assert list(v.tensor_offset) == [3 * 64 * 2 * 2048, 3 * 64 * 2 * 2048 + 64 * 2048]
    assert v.row_bytes == 2048 and v.tensor_count == 2 and v.heads == 8 and v.head_layout == kv.HND
    with pytest.raises(kv.KvError) as ei:
        lay.pool_view(0x1000, lay.total_byte_len, 32)
    assert ei.value.variant == "LayerOutOfRange"
    with pytest.raises(kv.KvError) as ei:
        lay.pool_view(0x1000, lay.total_byte_len, 0, kv.HND, 3)
    assert ei.value.variant == "InvalidArgument" and ei.value.name == "heads"
    mla = kv.PagedKvCacheLayout.new(kv.KvCacheRuntimeLayout.for_model("bf16", 64, 61, 1, 576, 1), 2)
    mv = mla.pool_view(0x1000, mla.total_byte_len, 60)
    assert mv.tensor_count == 1 and mv.row_bytes == 1152 and mv.tensor_offset[0] == 60 * 64 * 1152


def test_device_calls_fail_loudly_without_a_gpu():
    """On a host with no GPU the context cannot be created, and the error is
    a typed failure, not a silent fallback."""
    from sgl_rocm_kv import hip
    if hip.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(kv.KvError) as ei:
        kv.RocmKvPairCopyKernels(0)
    assert ei.value.variant in ("Hip", "InvalidArgument")


def test_synthetic_words_is_splitmix64():
    """The host copy of the fill stream against splitmix64's published
    first outputs for seed 0 (Vigna's reference implementation: state += the
    golden gamma, then the two xor-shift-multiply rounds)."""
    got = kv.synthetic_words(0, np.arange(3))
    assert [hex(int(x)) for x in got] == ["0xe220a8397b1dcdaf", "0x6e789e6aa1b965f4",
                                          "0x6c45d188009454f"]


# --- PD page-request descriptors (crates/sglang-srt/src/transfer.rs:1945-2090) ------------------

def test_remote_page_requests_golden(goldens):
    """crates/sglang-srt/tests/http_server.rs:2826-2833: a two-token prefill
    (page size 1) to a decode side advertising dst_kv_ptrs [0x9000],
    dst_kv_indices [4, 5], item length 128 -> target offsets 0x9000 + 4*128
    and 0x9000 + 5*128."""
    g = goldens["mooncake_remote_offsets"]
    reqs = kv.build_remote_page_requests(0x2000, g["item_len"], 2, 1, [0, 1], [g["dst_base"]],
                                         g["dst_kv_indices"], g["item_len"])
    assert list(reqs["target_offset"]) == g["target_offsets"]
    assert list(reqs["length"]) == [g["item_len"]] * 2
    assert list(reqs["source"]) == [0x2000, 0x2000 + g["item_len"]]


def test_page_requests_follow_the_span_page_offset():
    # token_offset 8 with page size 4 -> the span starts at target page 2
    reqs = kv.build_page_requests(0x1000, 256, 0x40000, 8, 6, 4, [7, 3])
    assert list(reqs["source"]) == [0x1000 + 7 * 256, 0x1000 + 3 * 256]
    assert list(reqs["target_offset"]) == [0x40000 + 2 * 256, 0x40000 + 3 * 256]


def test_remote_page_requests_place_every_split_of_every_page():
    """Execute the requests as byte copies on host buffers: split j of source
    page i must land at index dst_kv_indices[i] of decode buffer j."""
    rng = np.random.default_rng(2)
    PB, J, pages = 384, 3, 9
    item = PB // J
    base = 0x10_0000
    src = rng.integers(0, 256, 64 * PB, dtype=np.uint8)
    page_indices = rng.permutation(64)[:pages]
    dst_idx = rng.permutation(40)[:pages].astype(np.int32)
    ptrs = [0x4000_0000 + j * 0x100_0000 for j in range(J)]
    reqs = kv.build_remote_page_requests(base, PB, pages * 16 - 5, 16, page_indices, ptrs, dst_idx,
                                         item)
    assert len(reqs) == pages * J
    targets = [np.zeros(40 * item, np.uint8) for _ in range(J)]
    for r in reqs:
        j = max(i for i, p in enumerate(ptrs) if p <= r["target_offset"])
        off = int(r["target_offset"]) - ptrs[j]
        s0 = int(r["source"]) - base
        targets[j][off: off + int(r["length"])] = src[s0: s0 + int(r["length"])]
    for i, p in enumerate(page_indices):
        page = src[p * PB:(p + 1) * PB].reshape(J, item)
        for j in range(J):
            np.testing.assert_array_equal(targets[j][dst_idx[i] * item:(dst_idx[i] + 1) * item], page[j])


@pytest.mark.parametrize("args,variant,fields", [
    ((0x1000, 0, 2, 1, [0, 1], [0x9000], [4, 5], 128), "ZeroPageSize", None),
    ((0x1000, 128, 2, 1, [0, 1], [0x9000], [4, 5], 0), "ZeroRemoteKvItemSize", None),
    ((0x1000, 128, 2, 1, [0, 1], [], [4, 5], 128), "MissingRemoteKvPointers", None),
    ((0x1000, 128, 3, 2, [0], [0x9000], [4], 128), "SpanPageCountMismatch", (2, 1)),
    ((0x1000, 128, 2, 1, [0, 1], [0x9000], [4], 128), "RemoteKvIndexCountMismatch", (2, 1)),
    ((0x1000, 128, 2, 1, [0, 1], [0x9000, 0xA000], [4, 5], 128), "RemoteKvItemLayoutMismatch", (128, 256)),
    ((0x1000, 128, 2, 1, [0, 1], [0x9000], [4, -1], 128), "NegativeRemoteKvIndex", None),
    ((0x1000, 128, 1, 1, [2**60], [0x9000], [4], 128), "AddressOverflow", None),
    ((0x1000, 128, 1, 1, [0], [2**64 - 64], [4], 128), "OffsetOverflow", None),
])
def test_remote_page_request_errors(args, variant, fields):
    with pytest.raises(kv.KvError) as ei:
        kv.build_remote_page_requests(*args)
    assert ei.value.variant == variant
    if fields:
        assert ei.value.fields[:2] == fields
    if variant == "NegativeRemoteKvIndex":
        assert ei.value.fields[0] == 2**64 - 1


# --- page allocator (crates/sglang-srt/tests/cache_allocator.rs) ------------------------------

def test_allocator_returns_contiguous_free_pages_in_page_order():
    a = kv.CachePageAllocator(4)
    assert a.allocate(3) == [0, 1, 2]
    assert a.allocate(1) == [3]
    assert a.available_pages() == 0


def test_allocator_does_not_consume_pages_when_allocation_cannot_be_satisfied():
    a = kv.CachePageAllocator(2)
    with pytest.raises(kv.KvError) as ei:
        a.allocate(3)
    assert ei.value.variant == "OutOfSlots" and ei.value.fields[:2] == (3, 2)
    assert a.available_pages() == 2
    assert a.allocate(2) == [0, 1]


def test_allocator_reuses_released_pages_before_never_allocated_pages():
    a = kv.CachePageAllocator(5)
    allocated = a.allocate(3)
    a.release(allocated[1:])
    assert a.allocate(3) == [1, 2, 3]


def test_allocator_reset_restores_all_pages_in_page_order():
    a = kv.CachePageAllocator(4)
    a.allocate(3)
    a.reset()
    assert a.available_pages() == 4
    assert a.allocate(4) == [0, 1, 2, 3]


def test_page_aware_allocator_keeps_independent_requests_on_separate_pages():
    a = kv.CachePageAllocator.with_page_size(8, 4)
    assert a.allocate(3) == [0, 1, 2]
    assert a.allocate(2) == [4, 5]
    assert a.available_pages() == 0 and a.available_slots() == 0


def test_page_aware_allocator_extends_a_sequence_tail_before_reserving_another_page():
    a = kv.CachePageAllocator.with_page_size(8, 4)
    sequence = a.allocate(3)
    extension = a.allocate_for_sequence(sequence, 2)
    assert extension == [3, 4]
    sequence += extension
    a.release(extension)
    assert a.available_pages() == 1
    assert a.allocate(1) == [4]
    a.release(sequence[:3])
    assert a.available_pages() == 1


@pytest.mark.parametrize("cap,ps,variant,fields", [
    (8, 0, "ZeroPageSize", None), (0, 4, "ZeroSlotCapacity", None),
    (10, 4, "SlotCapacityNotPageAligned", (10, 4))])
def test_page_aware_allocator_rejects_invalid_pool_geometry(cap, ps, variant, fields):
    with pytest.raises(kv.KvError) as ei:
        kv.CachePageAllocator.with_page_size(cap, ps)
    assert ei.value.variant == variant
    if fields:
        assert ei.value.fields[:2] == fields


def test_allocator_slots_are_a_valid_transfer_plan():
    """Random allocate/release traffic: every allocation is distinct from
    every live slot, in range, and transfer_page_indices accepts each
    page-aligned allocation (slots contiguous within pages)."""
    rng = np.random.default_rng(4)
    P, cap = 16, 16 * 64
    a = kv.CachePageAllocator.with_page_size(cap, P)
    live = []
    for _ in range(400):
        if live and rng.random() < 0.4:
            victim = live.pop(int(rng.integers(0, len(live))))
            a.release(victim)
            continue
        n = int(rng.integers(1, 3 * P))
        try:
            slots = a.allocate(n)
        except kv.KvError as e:
            assert e.variant == "OutOfSlots"
            continue
        assert len(slots) == n and len(set(slots)) == n and max(slots) < cap
        used = {s for x in live for s in x}
        assert not used & set(slots)
        assert kv.transfer_page_indices(0, 0, slots, P) == [s // P for s in slots[::P]]
        live.append(slots)
    assert a.available_slots() + sum(-(-len(x) // P) * P for x in live) == cap


# --- span descriptor checksum (crates/sglang-srt/src/transfer.rs:548-570) ---------------------

def test_span_descriptor_checksum_golden(goldens):
    g = goldens["span_descriptor_checksum"]
    got = kv.transfer_span_checksum(g["request_id"], g["bootstrap_host"], g["bootstrap_port"],
                                    g["bootstrap_room"], g["data_parallel_rank"], g["token_offset"],
                                    g["token_count"], g["page_size"], g["cache_pages"],
                                    g["page_indices"])
    assert got == g["checksum"]


def test_sha256_matches_hashlib():
    import hashlib
    rng = np.random.default_rng(5)
    for n in [0, 1, 55, 56, 63, 64, 65, 119, 120, 1000, 4096 + 3]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert kv.sha256_hex(data) == hashlib.sha256(data).hexdigest(), n


@pytest.mark.parametrize("rows", [2**32 - 1, 2**32 - 4096 + 1, 2**40])
def test_row_counts_whose_last_tile_would_wrap_are_refused(rows):
    """The copy kernels index rows in 32 bits and the last tile of a launch
    must end below 2^32: the host refuses such row counts with a typed
    DimensionTooLarge before any device work (checked ahead of the context,
    so it holds on a host without a GPU)."""
    import ctypes
    v = kv.pool_view(0x1000, 1 << 40, page_size=1, page_stride_bytes=256, page_count=1 << 20,
                     tensor_offset=[0, 128], row_bytes=128, tensor_count=2)
    r = kv.rows_view([0x2000, 0x3000], [1 << 40, 1 << 40], [128, 128])
    slots = kv.device_buffer(0x4000, 1 << 40)
    lib = kv.lib()
    for rc in (lib.sgl_rocm_kv_pack_layer(None, ctypes.byref(v), ctypes.byref(slots), rows,
                                          ctypes.byref(r), None),
               lib.sgl_rocm_kv_unpack_layer(None, ctypes.byref(r), rows, ctypes.byref(v),
                                            ctypes.byref(slots), None),
               lib.sgl_rocm_kv_transfer_layer(None, ctypes.byref(v), ctypes.byref(slots), rows,
                                              ctypes.byref(v), ctypes.byref(slots), None)):
        assert kv.status_name(rc) == "DimensionTooLarge"
        d = kv._ErrorDetail()
        lib.sgl_kv_last_error(ctypes.byref(d))
        assert d.name == b"row_count" and d.a == rows and d.b == 2**32 - 1 - 4096


def test_header_compiles_as_c99_and_cpp17(tmp_path):
    """include/sgl_rocm_kv.h is the C ABI a binding generator or a C caller
    reads: it must compile on its own as strict C99 and as C++17, without a
    warning."""
    import shutil
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    inc = os.path.join(root, "include")
    for compiler, std, ext in (("gcc", "c99", "c"), ("g++", "c++17", "cpp")):
        if shutil.which(compiler) is None:
            pytest.skip(f"{compiler} not found")
        src = tmp_path / f"use_header.{ext}"
        src.write_text('#include "sgl_rocm_kv.h"\nint main(void) { return (int)sizeof(sgl_kv_pool_view) == 0; }\n')
        r = subprocess.run([compiler, f"-std={std}", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", inc,
                            "-c", str(src), "-o", str(tmp_path / f"use_header_{ext}.o")],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
