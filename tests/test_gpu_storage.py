"""GPU tests of the storage side of the boundary: the pool's device memory
(sgl_rocm_kv_storage_*, the ROCm counterpart of CudaKvStorage,
crates/sglang-srt/src/cuda_kv_cache.rs:170-509) and the descriptor the
transfer side registers (KvCacheMemoryProvider, :455-476).

The first two tests reproduce the reference's own acceptance tests of this
layer through the C ABI: cuda_backend_round_trips_page_major_device_kv_memory
(crates/sglang-srt/tests/cuda_backend.rs:251-322) and the KV-slot half of
cuda_runtime_kernels_execute_and_write_kv_slots (:462-495). Their expected
values are the reference's literals (tests/golden/reference_goldens.json).
The slot-map copies are checked against the oracle's literal restatement of
the reference's scatter/gather kernels (oracle/kv_oracle.c).
"""
import math

import numpy as np
import pytest

import oracle
import sgl_rocm_kv as kv
from sgl_rocm_kv import hip

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


def _runtime(goldens):
    rt = goldens["cuda_backend_slot_location"]["runtime"]
    return kv.KvCacheRuntimeLayout(rt["dtype"], rt["page_size"], rt["num_layers"], rt["kv_heads"],
                                   rt["head_dim"], rt["kv_tensors_per_token"], rt["bytes_per_token"],
                                   rt["page_size_bytes"])


def test_reference_page_major_round_trip(k, goldens):
    """cuda_backend.rs:251-322: a 16-page pool of the P16/L2/H8/D128 layout,
    page 3 written and read back, slot (1, 1, 63) at 522,240 / 2,048, one
    region of 2 MiB with 131,072-byte pages located on this device, a decode
    remote layout of item length 131,072, and device memory taken by the
    pool and given back when it is dropped."""
    _say("reference page-major round trip")
    g = goldens["cuda_backend_page_round_trip"]
    free_before, total = k.memory_info()
    assert 0 < free_before <= total
    pool = kv.allocate_rocm_kv_cache(k, _runtime(goldens), g["page_count"])
    layout = pool.layout()
    psb = layout.runtime.page_size_bytes
    assert psb == g["page_size_bytes"]
    # a fresh pool is zero-filled (CudaKvStorage::allocate fills 0)
    assert not pool.storage().read_page(layout, g["page_index"]).any()
    pattern = (np.arange(psb) % g["pattern_modulus"]).astype(np.uint8)
    pool.storage_mut().write_page(layout, g["page_index"], pattern)
    np.testing.assert_array_equal(pool.storage().read_page(layout, g["page_index"]), pattern)
    # the neighbouring pages are untouched
    for p in (g["page_index"] - 1, g["page_index"] + 1):
        assert not pool.storage().read_page(layout, p).any()

    sl = g["slot_location"]
    loc = pool.storage().slot_location(layout, sl["layer"], sl["tensor"], sl["slot"])
    assert (loc.byte_offset, loc.byte_len) == (sl["byte_offset"], sl["byte_len"])
    assert loc.device_ptr == pool.storage().device_ptr + loc.byte_offset

    mem = pool.transferable_kv_cache_memory()
    assert len(mem.regions()) == g["regions"]
    assert mem.page_size_bytes() == g["page_size_bytes"]
    assert mem.location() == (kv.LOCATION_ROCM, k.device)
    assert mem.location_label() == f"hip:{k.device}"
    assert mem.regions()[0].byte_len == g["region_byte_len"]
    assert mem.regions()[0].base_addr == pool.storage().device_ptr
    remote = mem.mooncake_decode_remote_layout(g["decode_remote_layout_indices"])
    assert remote.dst_kv_item_len == g["dst_kv_item_len"]
    assert remote.dst_kv_ptrs == [pool.storage().device_ptr]

    free_after, _ = k.memory_info()
    assert free_after < free_before
    pool.close()
    free_released, _ = k.memory_info()
    assert free_released > free_after


def test_reference_tensor_slot_round_trip(k, goldens):
    """cuda_backend.rs:462-495: a 2-page pool, slot 7 of layer 1, tensor 0
    written from one device allocation and read into another (device to
    device), bytes offset % 251."""
    _say("reference tensor-slot round trip")
    g = goldens["cuda_backend_tensor_slot_round_trip"]
    pool = kv.allocate_rocm_kv_cache(k, _runtime(goldens), g["page_count"])
    layout = pool.layout()
    n = layout.bytes_per_token_per_tensor
    assert n == g["slot_byte_len"]
    pattern = (np.arange(n) % g["pattern_modulus"]).astype(np.uint8)
    src, dst = hip.DeviceBuffer.from_array(pattern), hip.DeviceBuffer(n)
    dst.fill(0)
    pool.storage_mut().write_tensor_slot_from_device(layout, g["layer"], g["tensor"], g["slot"], src, 0)
    pool.storage().read_tensor_slot_to_device(layout, g["layer"], g["tensor"], g["slot"], dst, 0)
    hip.synchronize()
    np.testing.assert_array_equal(dst.download(), pattern)
    # exactly that range of the pool changed, where the oracle's layout puts it
    rt = layout.runtime
    lay = oracle.layout(rt.page_size, rt.num_layers, rt.kv_tensors_per_token, rt.bytes_per_token,
                        rt.page_size_bytes, g["page_count"])
    rc, (s, e) = oracle.tensor_slot_byte_range(lay, g["layer"], g["tensor"], g["slot"])
    assert rc == 0
    whole = np.concatenate([pool.storage().read_page(layout, p) for p in range(g["page_count"])])
    np.testing.assert_array_equal(whole[s:e], pattern)
    assert not np.delete(whole, np.arange(s, e)).any()
    pool.close()


def test_slot_map_copies_match_the_reference_kernels(k, goldens):
    """write_kv_slots_from_device / read_kv_slots_to_device (cuda_kv_cache.rs:
    296-374) through an uploaded slot map, with strided rows, against the
    oracle's literal restatement of sglang_scatter/gather_kv_pair_bytes."""
    _say("slot-map scatter/gather through the storage")
    from kvmath import acceptance_rows, strided_rows
    pool = kv.allocate_rocm_kv_cache(k, _runtime(goldens), 6)
    layout = pool.layout()
    rng = np.random.default_rng(7)
    slots = rng.choice(layout.slot_count, size=37, replace=False).astype(np.uint64)
    smap = pool.storage().upload_slot_map(layout, slots)
    assert len(smap) == 37
    np.testing.assert_array_equal(smap.slots(), slots)
    np.testing.assert_array_equal(hip_download_u64(smap.allocation(), 37), slots)
    for layer in range(layout.runtime.num_layers):
        geo = layout.kv_pair_copy_geometry(layer)
        rb = geo.row_bytes
        ks, vs = rb + 48, rb + 16
        keys_h, exp_k = acceptance_rows(37, rb, ks, 11 + layer)
        values_h, exp_v = acceptance_rows(37, rb, vs, 23 + layer)
        keys, values = hip.DeviceBuffer.from_array(keys_h), hip.DeviceBuffer.from_array(values_h)
        before = np.concatenate([pool.storage().read_page(layout, p) for p in range(6)])
        pool.storage_mut().write_kv_slots_from_device(k, layout, layer, smap, keys=keys, key_row_stride_bytes=ks,
                                                      values=values, value_row_stride_bytes=vs)
        got = np.concatenate([pool.storage().read_page(layout, p) for p in range(6)])
        want = before.copy()
        assert oracle.ref_scatter_kv_pair_bytes(
            keys_h, values_h, slots, want, slot_count=layout.slot_count, page_size=geo.page_size,
            page_stride_bytes=geo.page_stride_bytes, key_in_page_offset=geo.key_in_page_offset,
            value_in_page_offset=geo.value_in_page_offset, row_bytes=rb, key_row_stride_bytes=ks,
            value_row_stride_bytes=vs) == 0
        np.testing.assert_array_equal(got, want)
        gk, gv = hip.DeviceBuffer(37 * rb), hip.DeviceBuffer(37 * rb)
        gk.fill(0)
        gv.fill(0)
        pool.storage().read_kv_slots_to_device(k, layout, layer, smap, keys=gk, key_row_stride_bytes=rb,
                                               values=gv, value_row_stride_bytes=rb)
        np.testing.assert_array_equal(strided_rows(gk.download(), 37, rb, rb), np.stack(exp_k))
        np.testing.assert_array_equal(strided_rows(gv.download(), 37, rb, rb), np.stack(exp_v))
    smap.close()
    pool.clear()
    assert not any(pool.storage().read_page(layout, p).any() for p in range(6))
    pool.close()


def hip_download_u64(b, n):
    out = np.zeros(n, np.uint64)
    hip.check(hip.lib().hipMemcpy(out.ctypes.data, b.ptr, n * 8, 2), "hipMemcpy")
    return out


def test_storage_errors_mirror_the_reference(k, goldens):
    """validate_layout / validate_slot_map / page buffer checks (cuda_kv_cache.rs:
    224-256, 391-421) and CudaContext::allocate's ZeroAllocation (cuda.rs:477-480)."""
    _say("storage error variants")
    rt = _runtime(goldens)
    with pytest.raises(kv.KvError) as ei:
        kv.RocmKvStorage.allocate(k, 0, rt.page_size_bytes)
    assert ei.value.variant == "ZeroAllocation"
    pool = kv.allocate_rocm_kv_cache(k, rt, 4)
    layout = pool.layout()
    other = kv.PagedKvCacheLayout.new(rt, 5)
    with pytest.raises(kv.KvError) as ei:
        pool.storage().read_page(other, 0)
    assert ei.value.variant == "StorageSizeMismatch"
    assert ei.value.fields[:2] == (other.total_byte_len, layout.total_byte_len)
    with pytest.raises(kv.KvError) as ei:
        pool.storage_mut().write_page(layout, 0, np.zeros(rt.page_size_bytes - 1, np.uint8))
    assert ei.value.variant == "PageBufferSizeMismatch"
    assert ei.value.fields[:2] == (rt.page_size_bytes, rt.page_size_bytes - 1)
    with pytest.raises(kv.KvError) as ei:
        pool.storage().read_page(layout, 4)
    assert ei.value.variant == "PageOutOfRange"
    # a storage whose page size differs from the layout's: PageBufferSizeMismatch
    odd = kv.RocmKvStorage.allocate(k, layout.total_byte_len, rt.page_size_bytes // 2)
    with pytest.raises(kv.KvError) as ei:
        odd.validate_layout(layout)
    assert ei.value.variant == "PageBufferSizeMismatch"
    odd.close()
    # a region that is not a whole number of pages cannot be described
    ragged = kv.RocmKvStorage.allocate(k, 3 * 4096 + 1, 4096)
    with pytest.raises(kv.KvError) as ei:
        ragged.transferable_kv_cache_memory()
    assert ei.value.variant == "Descriptor"
    ragged.close()
    with pytest.raises(kv.KvError) as ei:
        pool.storage().upload_slot_map(layout, [])
    assert ei.value.variant == "EmptySlotMap"
    with pytest.raises(kv.KvError) as ei:
        pool.storage().upload_slot_map(layout, [0, layout.slot_count])
    assert ei.value.variant == "BatchSlotOutOfRange"
    assert ei.value.fields == (1, layout.slot_count, layout.slot_count)
    # a map validated for another slot count: SlotMapCapacityMismatch
    bigger = kv.allocate_rocm_kv_cache(k, rt, 8)
    smap = bigger.storage().upload_slot_map(bigger.layout(), [1, 2])
    rb = layout.bytes_per_token_per_tensor
    rows = hip.DeviceBuffer(2 * rb)
    with pytest.raises(kv.KvError) as ei:
        pool.storage_mut().write_kv_slots_from_device(k, layout, 0, smap, keys=rows, key_row_stride_bytes=rb,
                                                      values=rows, value_row_stride_bytes=rb)
    assert ei.value.variant == "SlotMapCapacityMismatch"
    assert ei.value.fields[:2] == (bigger.layout().slot_count, layout.slot_count)
    # a slot source too short for the slot: AllocationOutOfBounds
    short = hip.DeviceBuffer(rb - 1)
    with pytest.raises(kv.KvError) as ei:
        pool.storage_mut().write_tensor_slot_from_device(layout, 0, 0, 0, short, 0)
    assert ei.value.variant == "AllocationOutOfBounds"
    # a host buffer is not on the device: DeviceMismatch
    pinned = hip.PinnedBuffer(rb)
    with pytest.raises(kv.KvError) as ei:
        pool.storage_mut().write_tensor_slot_from_device(layout, 0, 0, 0, kv.device_buffer(pinned.ptr, rb), 0)
    assert ei.value.variant == "DeviceMismatch"
    smap.close()
    bigger.close()
    pool.close()


def test_storage_pools_drive_the_transfer_backend(k):
    """A prefill pool and a decode pool obtained from the storage ABI (no
    caller allocation) registered with the transfer backend: one span moves,
    and the decode pool's bytes match the oracle's transfer of the same
    prefill bytes."""
    _say("storage pools through the transfer backend")
    P_SRC, P_DST, L, H, D = 1, 16, 3, 2, 64
    rb = H * D * 2
    src_rt = kv.KvCacheRuntimeLayout("bf16", P_SRC, L, H, D, 2, L * 2 * rb, P_SRC * L * 2 * rb)
    dst_rt = kv.KvCacheRuntimeLayout("bf16", P_DST, L, H, D, 2, L * 2 * rb, P_DST * L * 2 * rb)
    prefill = kv.allocate_rocm_kv_cache(k, src_rt, 256)
    decode = kv.allocate_rocm_kv_cache(k, dst_rt, 16)
    buf = prefill.storage().allocation()
    k.fill_synthetic(buf, 99)
    hip.synchronize()
    be = kv.RocmKvTransferBackend(k, kv.BACKEND_DIRECT, max_rows=1024)
    be.register_pools(prefill, decode)
    rng = np.random.default_rng(3)
    slots = rng.choice(256, size=40, replace=False).astype(np.uint64)
    table = np.array([5, 2, 9], np.int32)
    be.submit(7, "c" * 64, 0, slots, table)
    be.wait()
    events, pending = be.poll()
    assert pending == 0 and len(events) == 1 and events[0].status == 0
    src_bytes = np.concatenate([prefill.storage().read_page(prefill.layout(), p) for p in range(256)])
    got = np.concatenate([decode.storage().read_page(decode.layout(), p) for p in range(16)])
    # expected: the oracle's pool-to-pool transfer, layer by layer, over the
    # oracle's own layout arithmetic and span resolution
    src_lay = oracle.layout(P_SRC, L, 2, src_rt.bytes_per_token, src_rt.page_size_bytes, 256)
    dst_lay = oracle.layout(P_DST, L, 2, dst_rt.bytes_per_token, dst_rt.page_size_bytes, 16)
    want = np.zeros_like(got)
    for layer in range(L):
        def pool(lay, rt, pages):
            offs = tuple(oracle.tensor_token_byte_range(lay, 0, layer, t, 0)[1][0] for t in range(2))
            return oracle.Pool(rt.page_size, rt.page_size_bytes, pages, offs, rb, 2, H, False)
        sp, dp = pool(src_lay, src_rt, 256), pool(dst_lay, dst_rt, 16)
        spans = np.array([(0, 0, 40, 0)], dtype=oracle.SPAN_DTYPE)
        dst_slots, flag = oracle.resolve_slots(dp, 40, page_table=table, spans=spans)
        assert flag == 0
        oracle.transfer(sp, src_bytes, slots, dp, want, dst_slots)
    np.testing.assert_array_equal(got, want)
    be.shutdown()
    be.close()
    decode.close()
    prefill.close()


def _bf16(values) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (the reference's test helper,
    crates/sglang-srt/tests/cuda_backend.rs:125-129, restated by the oracle)."""
    return oracle.f32_to_bf16(np.asarray(values, np.float32))


def test_reference_attention_over_physical_slots(k):
    """cuda_bf16_paged_attention_reads_mooncake_registered_physical_kv_slots
    (cuda_backend.rs:641-781): a scheduler's two-request prefill ([10, 11, 12]
    and [20, 21] from a fresh 8-slot page allocator, page size 1) gives causal
    metadata over its physical slots; keys (i - 11) * 0.03125 and values
    (17 - i) * 0.046875 go into a 2-page P4 L1 H2 D4 pool through an uploaded
    slot map (write_kv_slots_from_device); queries ((7 i mod 29) - 14) *
    0.0625, 4 query heads, scale 1/2. The attention reads the very allocation
    the Mooncake descriptor registers. Checked against the float64 oracle
    within the reference's 0.02 and within bf16 rounding of the output."""
    _say("reference attention over physical slots")
    P, L, H, D, qh = 4, 1, 2, 4, 4
    rt = kv.KvCacheRuntimeLayout("bf16", P, L, H, D, 2, L * H * D * 2 * 2, P * L * H * D * 2 * 2)
    pool = kv.allocate_rocm_kv_cache(k, rt, 2)
    layout = pool.layout()
    # the scheduler's slots: CachePageAllocator::new(8) hands out 0, 1, 2 then 3, 4
    alloc = kv.CachePageAllocator(8, 1)
    a = alloc.allocate_for_sequence([], 3)
    b = alloc.allocate_for_sequence([], 2)
    slots = np.concatenate([a, b]).astype(np.uint64)
    np.testing.assert_array_equal(slots, np.arange(5))
    qri = np.array([0, 0, 0, 1, 1], np.uint32)       # one query per prefill token
    qsl = np.array([1, 2, 3, 1, 2], np.uint64)       # causal: position + 1
    rso = np.array([0, 3, 5], np.uint64)
    smap = pool.storage().upload_slot_map(layout, slots)
    n = len(slots) * H * D
    keys_h = _bf16((np.arange(n) - 11.0) * 0.03125)
    values_h = _bf16((17.0 - np.arange(n)) * 0.046875)
    row = H * D * 2
    keys, values = hip.DeviceBuffer.from_array(keys_h), hip.DeviceBuffer.from_array(values_h)
    pool.storage_mut().write_kv_slots_from_device(k, layout, 0, smap, keys=keys, key_row_stride_bytes=row,
                                                  values=values, value_row_stride_bytes=row)
    q_h = _bf16(((np.arange(5 * qh * D) * 7 % 29) - 14.0) * 0.0625)
    mem = pool.transferable_kv_cache_memory()
    assert mem.regions()[0].base_addr == pool.storage().device_ptr
    plan = kv.PagedAttentionPlan.for_layer(layout, 0, 5, 2, 5, qh, 1.0 / math.sqrt(D))
    out = hip.DeviceBuffer(plan.output_required_bytes)
    k.paged_attention(plan, queries=hip.DeviceBuffer.from_array(q_h),
                      query_request_indices=hip.DeviceBuffer.from_array(qri),
                      query_sequence_lengths=hip.DeviceBuffer.from_array(qsl),
                      request_slot_offsets=hip.DeviceBuffer.from_array(rso),
                      sequence_slots=hip.DeviceBuffer.from_array(slots),
                      pool=pool.storage().allocation(), output=out)
    got = oracle.bf16_to_f32(out.download().view(np.uint16)).reshape(5, qh, D)
    pool_bytes = np.concatenate([pool.storage().read_page(layout, p) for p in range(2)])
    want, flags = oracle.paged_attention(
        pool_bytes, q_h.reshape(5, qh, D), qri, qsl, rso, slots, page_size=P,
        page_stride=plan.page_stride_bytes, key_offset=plan.key_in_page_offset,
        value_offset=plan.value_in_page_offset, kv_heads=H, dk=D, dv=D, scale=1.0 / math.sqrt(D),
        slot_count=layout.slot_count, hnd=False)
    assert flags == 0
    err = np.abs(got - want)
    assert err.max() <= 0.02                                        # the reference's tolerance
    assert (err <= 2.0 ** -8 * np.abs(want) + 1e-3).all(), err.max()  # bf16 rounding of the output
    smap.close()
    pool.close()


def test_reference_asymmetric_compressed_mla(k):
    """cuda_bf16_paged_attention_executes_asymmetric_compressed_mla_kv
    (cuda_backend.rs:783-882): a 1-page P4 pool of the tensor-pair layout with
    3-dim keys (6 bytes) and 2-dim values (4 bytes); slot 0 holds key [1, 0, 0]
    and value [10, 20], slot 1 key [0, 1, 0] and value [30, 40], each written
    with write_tensor_slot_from_device; one query [1, 0, 0] over both slots
    (for_single_query), scale 1. The output is w [10, 20] + (1 - w) [30, 40]
    with w = e / (e + 1): within the reference's 0.05, and within the bf16
    rounding of the output."""
    _say("reference asymmetric compressed MLA")
    rt = kv.KvCacheRuntimeLayout("bf16", 4, 1, 1, 3, 2, 10, 40)
    layout = kv.PagedKvCacheLayout.new_with_tensor_pair(rt, 1, 6, 4)
    storage = kv.RocmKvStorage.allocate(k, layout.total_byte_len, layout.runtime.page_size_bytes)
    for slot, key, value in ((0, [1.0, 0.0, 0.0], [10.0, 20.0]), (1, [0.0, 1.0, 0.0], [30.0, 40.0])):
        kb, vb = hip.DeviceBuffer.from_array(_bf16(key)), hip.DeviceBuffer.from_array(_bf16(value))
        storage.write_tensor_slot_from_device(layout, 0, 0, slot, kb, 0)
        storage.write_tensor_slot_from_device(layout, 0, 1, slot, vb, 0)
        hip.synchronize()
    slots = np.array([0, 1], np.uint64)            # CudaPagedAttentionMetadata::for_single_query
    plan = kv.PagedAttentionPlan.for_layer(layout, 0, 1, 1, 2, 1, 1.0)
    assert (plan.key_row_bytes, plan.value_row_bytes) == (6, 4)
    out = hip.DeviceBuffer(plan.output_required_bytes)
    k.paged_attention(plan, queries=hip.DeviceBuffer.from_array(_bf16([1.0, 0.0, 0.0])),
                      query_request_indices=hip.DeviceBuffer.from_array(np.zeros(1, np.uint32)),
                      query_sequence_lengths=hip.DeviceBuffer.from_array(np.array([2], np.uint64)),
                      request_slot_offsets=hip.DeviceBuffer.from_array(np.array([0, 2], np.uint64)),
                      sequence_slots=hip.DeviceBuffer.from_array(slots), pool=storage.allocation(), output=out)
    got = oracle.bf16_to_f32(out.download().view(np.uint16))
    w = math.e / (math.e + 1.0)
    want = np.array([w * 10 + (1 - w) * 30, w * 20 + (1 - w) * 40])
    assert np.abs(got - want).max() <= 0.05                          # the reference's tolerance
    assert (np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-3).all(), (got, want)
    storage.close()


def test_placed_allocation_keeps_the_fastest_candidate(k):
    """sgl_rocm_kv_storage_allocate_placed (no counterpart in the reference):
    three allocations probed with one layer's unpack, the fastest kept,
    zero-filled and of the requested size, the others given back; the kept
    pool is an ordinary pool (an unpack into it equals the oracle's)."""
    _say("placed allocation")
    P, L, H, D, pages = 64, 2, 8, 128, 128
    rb = H * D * 2
    rt = kv.KvCacheRuntimeLayout("bf16", P, L, H, D, 2, L * 2 * rb, P * L * 2 * rb)
    layout = kv.PagedKvCacheLayout.new(rt, pages)
    nbytes, psb = layout.total_byte_len, rt.page_size_bytes
    rows_n = 3000
    probe_rows = hip.DeviceBuffer(rows_n * 2 * rb)
    k.fill_synthetic(kv.device_buffer(probe_rows.ptr, probe_rows.nbytes), 11)
    hip.synchronize()
    view = layout.pool_view(0, nbytes, 1)
    free_before, _ = k.memory_info()
    storage, rep = kv.RocmKvStorage.allocate_placed(k, nbytes, psb, view,
                                                    kv.device_buffer(probe_rows.ptr, probe_rows.nbytes), 3)
    free_after, _ = k.memory_info()
    _say(f"placement report {rep}")
    assert rep["candidates"] == 3 and rep["probe_rows"] == rows_n
    assert len(rep["probe_us"]) == 3 and min(rep["probe_us"]) > 0
    assert rep["probe_us"][rep["chosen"]] == min(rep["probe_us"])
    assert storage.byte_len() == nbytes and storage.page_size_bytes() == psb
    # one pool's worth held (allocation granularity aside), not three
    assert nbytes // 2 <= free_before - free_after < 2 * nbytes
    whole = np.concatenate([storage.read_page(layout, p) for p in range(pages)])
    assert not whole.any(), "the kept pool is zero-filled after the probe"

    # an ordinary pool: unpack rows into layer 0 and compare with the oracle
    rng = np.random.default_rng(5)
    n = 777
    slots = rng.choice(layout.slot_count, size=n, replace=False).astype(np.uint64)
    rows = rng.integers(0, 256, size=(2, n, rb), dtype=np.uint8)
    rows_dev = hip.DeviceBuffer.from_array(rows)
    slots_dev = hip.DeviceBuffer.from_array(slots)
    b = storage.allocation()
    rv = kv.rows_view([rows_dev.ptr, rows_dev.ptr + n * rb], [n * rb, n * rb], [rb, rb])
    k.unpack_layer(rv, n, layout.pool_view(b.ptr, b.byte_len, 0), kv.device_buffer(slots_dev.ptr, slots_dev.nbytes))
    hip.synchronize()
    k.check_errors()
    got = np.concatenate([storage.read_page(layout, p) for p in range(pages)])
    offs = tuple(layout.pool_view(0, nbytes, 0).tensor_offset[t] for t in range(2))
    pool = oracle.Pool(P, psb, pages, offs, rb, 2, H, False)
    want = np.zeros(nbytes, np.uint8)
    oracle.unpack(pool, want, slots, rows[0], rows[1], rb, rb)
    np.testing.assert_array_equal(got, want)
    storage.close()
    free_released, _ = k.memory_info()
    assert free_released > free_after


def test_placed_allocation_errors(k):
    """Candidate counts outside 1..8, probe rows too small for one row and a
    missing view are refused before anything is allocated."""
    _say("placed allocation errors")
    P, L, H, D = 16, 1, 2, 64
    rb = H * D * 2
    rt = kv.KvCacheRuntimeLayout("bf16", P, L, H, D, 2, L * 2 * rb, P * L * 2 * rb)
    layout = kv.PagedKvCacheLayout.new(rt, 4)
    nbytes = layout.total_byte_len
    rows = hip.DeviceBuffer(4 * 2 * rb)
    view = layout.pool_view(0, nbytes, 0)
    db = kv.device_buffer(rows.ptr, rows.nbytes)
    for bad in (0, 9):
        with pytest.raises(kv.KvError) as e:
            kv.RocmKvStorage.allocate_placed(k, nbytes, rt.page_size_bytes, view, db, bad)
        assert e.value.code == kv.INVALID_ARGUMENT and e.value.name == "candidates"
    with pytest.raises(kv.KvError) as e:
        kv.RocmKvStorage.allocate_placed(k, nbytes, rt.page_size_bytes, view,
                                         kv.device_buffer(rows.ptr, 2 * rb - 1), 2)
    assert e.value.code == kv.INVALID_ARGUMENT and e.value.name == "probe_rows"
    with pytest.raises(kv.KvError) as e:
        kv.RocmKvStorage.allocate_placed(k, 0, rt.page_size_bytes, view, db, 2)
    assert e.value.code == kv.ZERO_ALLOCATION
    # probe rows in host memory are not the context's device memory
    host = np.zeros(4 * 2 * rb, np.uint8)
    with pytest.raises(kv.KvError) as e:
        kv.RocmKvStorage.allocate_placed(k, nbytes, rt.page_size_bytes, view,
                                         kv.device_buffer(host.ctypes.data, host.nbytes), 2)
    assert e.value.variant == "DeviceMismatch" and e.value.name == "probe_rows"
    # a single candidate is an ordinary probed allocation
    storage, rep = kv.RocmKvStorage.allocate_placed(k, nbytes, rt.page_size_bytes, view, db, 1)
    assert rep["candidates"] == 1 and rep["chosen"] == 0 and rep["probe_rows"] == 4
    assert storage.byte_len() == nbytes
    storage.close()


@pytest.mark.parametrize("form", ["pair", "packed", "hnd", "fp8"])
def test_placed_allocation_probes_every_pool_form(k, form):
    """The placement probe packs and unpacks through the view it is given:
    DeepSeek-V3's key/value pair of unequal widths (1,152 / 1,024 B), the
    649-byte packed-MLA rows (the byte-realigning kernels), head-major pages
    and fp8 rows whose view carries a per-layer scale (the probe moves bytes
    only and leaves the scale alone). Each kept pool is zero-filled and
    round-trips rows (and the scale)."""
    _say(f"placed allocation, {form} view")
    P, L, pages = 16, 2, 64
    if form == "pair":
        kb, vb, T, H, hl = 1152, 1024, 2, 1, kv.NHD
    elif form == "packed":
        kb, vb, T, H, hl = 649, 0, 1, 1, kv.NHD
    elif form == "fp8":
        kb, vb, T, H, hl = 576, 0, 1, 1, kv.NHD
    else:
        kb, vb, T, H, hl = 1024, 1024, 2, 8, kv.HND
    token = kb + vb
    stride = P * L * token
    nbytes = pages * stride
    pool_scale = hip.DeviceBuffer.from_array(np.array([-7.0], np.float32))

    def view(base):
        return kv.pool_view(base, nbytes, page_size=P, page_stride_bytes=stride, page_count=pages,
                            tensor_offset=[0, P * kb][:T], row_bytes=kb, tensor_count=T, heads=H,
                            head_layout=hl, value_row_bytes=vb if form == "pair" else 0,
                            scale=pool_scale.ptr if form == "fp8" else None)

    probe = hip.DeviceBuffer(600 * token)
    storage, rep = kv.RocmKvStorage.allocate_placed(k, nbytes, stride, view(0),
                                                    kv.device_buffer(probe.ptr, probe.nbytes), 2)
    assert rep["candidates"] == 2 and rep["probe_rows"] == 600 and min(rep["probe_us"]) > 0
    b = storage.allocation()
    assert b.byte_len == nbytes
    whole = np.zeros(nbytes, np.uint8)
    hip.memcpy_async(whole.ctypes.data, b.ptr, nbytes, "d2h")
    hip.synchronize()
    assert not whole.any()
    rng = np.random.default_rng(9)
    n = 300
    slots = rng.choice(P * pages, size=n, replace=False).astype(np.uint64)
    widths = [kb, vb][:T]
    rows = [rng.integers(0, 256, size=n * w, dtype=np.uint8) for w in widths]
    src = [hip.DeviceBuffer.from_array(r) for r in rows]
    back = [hip.DeviceBuffer(n * w) for w in widths]
    sd = hip.DeviceBuffer.from_array(slots)
    sdb = kv.device_buffer(sd.ptr, sd.nbytes)
    # the probe left the pool's scale as it was
    np.testing.assert_array_equal(pool_scale.download(dtype=np.float32), [-7.0])
    rows_scale = hip.DeviceBuffer.from_array(np.array([0.375], np.float32))
    back_scale = hip.DeviceBuffer.from_array(np.array([0.0], np.float32))
    fp8 = form == "fp8"
    k.unpack_layer(kv.rows_view([x.ptr for x in src], [n * w for w in widths], widths,
                                rows_scale.ptr if fp8 else None), n, view(b.ptr), sdb)
    k.pack_layer(view(b.ptr), sdb, n, kv.rows_view([x.ptr for x in back], [n * w for w in widths], widths,
                                                   back_scale.ptr if fp8 else None))
    hip.synchronize()
    k.check_errors()
    for r, x in zip(rows, back):
        np.testing.assert_array_equal(x.download(), r)
    if fp8:
        np.testing.assert_array_equal(pool_scale.download(dtype=np.float32), [0.375])
        np.testing.assert_array_equal(back_scale.download(dtype=np.float32), [0.375])
    storage.close()


def test_placed_allocation_probes_pool_to_pool(k):
    """With a source pool's view instead of probe rows, each candidate is
    timed on a pool-to-pool transfer from it; the source is only read, and
    the kept pool then takes a transfer whose bytes equal the oracle's."""
    _say("placed allocation, pool-to-pool probe")
    L, H, D = 2, 2, 64
    rb = H * D * 2
    src_rt = kv.KvCacheRuntimeLayout("bf16", 1, L, H, D, 2, L * 2 * rb, L * 2 * rb)
    dst_rt = kv.KvCacheRuntimeLayout("bf16", 16, L, H, D, 2, L * 2 * rb, 16 * L * 2 * rb)
    src_l, dst_l = kv.PagedKvCacheLayout.new(src_rt, 4096), kv.PagedKvCacheLayout.new(dst_rt, 128)
    src = kv.RocmKvStorage.allocate(k, src_l.total_byte_len, src_rt.page_size_bytes)
    sb = src.allocation()
    k.fill_synthetic(sb, 31)
    hip.synchronize()
    before = np.zeros(sb.byte_len, np.uint8)
    hip.memcpy_async(before.ctypes.data, sb.ptr, sb.byte_len, "d2h")
    hip.synchronize()
    with pytest.raises(kv.KvError) as e:   # neither rows nor a source to probe with
        kv.RocmKvStorage.allocate_placed(k, dst_l.total_byte_len, dst_rt.page_size_bytes,
                                         dst_l.pool_view(0, dst_l.total_byte_len, 0), None, 2)
    assert e.value.code == kv.INVALID_ARGUMENT and e.value.name == "probe_rows"
    dst, rep = kv.RocmKvStorage.allocate_placed(
        k, dst_l.total_byte_len, dst_rt.page_size_bytes, dst_l.pool_view(0, dst_l.total_byte_len, 0), None, 3,
        probe_source=src_l.pool_view(sb.ptr, sb.byte_len, 0))
    _say(f"placement report {rep}")
    assert rep["candidates"] == 3 and rep["probe_rows"] == 2048 and min(rep["probe_us"]) > 0
    assert rep["probe_us"][rep["chosen"]] == min(rep["probe_us"])
    after = np.zeros(sb.byte_len, np.uint8)
    hip.memcpy_async(after.ctypes.data, sb.ptr, sb.byte_len, "d2h")
    hip.synchronize()
    np.testing.assert_array_equal(after, before)   # the probe only read the source
    db = dst.allocation()
    got0 = np.zeros(db.byte_len, np.uint8)
    hip.memcpy_async(got0.ctypes.data, db.ptr, db.byte_len, "d2h")
    hip.synchronize()
    assert not got0.any()
    rng = np.random.default_rng(13)
    n = 500
    s_slots = rng.choice(4096, size=n, replace=False).astype(np.uint64)
    d_slots = rng.choice(2048, size=n, replace=False).astype(np.uint64)
    ss, ds = hip.DeviceBuffer.from_array(s_slots), hip.DeviceBuffer.from_array(d_slots)
    for layer in range(L):
        k.transfer_layer(src_l.pool_view(sb.ptr, sb.byte_len, layer), kv.device_buffer(ss.ptr, ss.nbytes), n,
                         dst_l.pool_view(db.ptr, db.byte_len, layer), kv.device_buffer(ds.ptr, ds.nbytes))
    hip.synchronize()
    k.check_errors()
    got = np.zeros(db.byte_len, np.uint8)
    hip.memcpy_async(got.ctypes.data, db.ptr, db.byte_len, "d2h")
    hip.synchronize()
    src_lay = oracle.layout(1, L, 2, src_rt.bytes_per_token, src_rt.page_size_bytes, 4096)
    dst_lay = oracle.layout(16, L, 2, dst_rt.bytes_per_token, dst_rt.page_size_bytes, 128)
    want = np.zeros_like(got)
    for layer in range(L):
        def pool(lay, rt, pages):
            offs = tuple(oracle.tensor_token_byte_range(lay, 0, layer, t, 0)[1][0] for t in range(2))
            return oracle.Pool(rt.page_size, rt.page_size_bytes, pages, offs, rb, 2, H, False)
        oracle.transfer(pool(src_lay, src_rt, 4096), before, s_slots, pool(dst_lay, dst_rt, 128), want, d_slots)
    np.testing.assert_array_equal(got, want)
    dst.close()
    src.close()
