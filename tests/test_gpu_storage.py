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
