"""Host tests of the storage side of the C ABI that need no GPU: the memory
location labels Mooncake registers pools under
(mooncake_memory_location_label, crates/sglang-srt/src/transfer.rs:1662-1676),
the decode remote layout derived from a memory descriptor
(mooncake_decode_remote_layout, transfer.rs:1693-1703, pinned by
crates/sglang-srt/tests/cuda_backend.rs:304-309), and the NULL handling of
the storage entry points (no HIP call is made for them)."""
import ctypes

import pytest

import sgl_rocm_kv as kv


@pytest.mark.parametrize("kind, device, label", [
    (kv.LOCATION_CPU, 0, "cpu:0"),
    (kv.LOCATION_CUDA, 2, "cuda:2"),
    (kv.LOCATION_ROCM, 0, "hip:0"),
    (kv.LOCATION_ROCM, 7, "hip:7"),
    (kv.LOCATION_MUSA, 1, "musa:1"),
    (kv.LOCATION_NPU, 3, "npu:3"),
])
def test_memory_location_labels(kind, device, label):
    assert kv.memory_location_label(kind, device) == label


@pytest.mark.parametrize("kind", [kv.LOCATION_METAL, kv.LOCATION_XPU, kv.LOCATION_HPU])
def test_unsupported_memory_locations(kind):
    with pytest.raises(kv.KvError) as ei:
        kv.memory_location_label(kind, 0)
    assert ei.value.variant == "UnsupportedMemoryLocation"
    assert ei.value.fields[0] == kind
    assert "does not support KV memory location" in ei.value.message


def test_unknown_location_kind_is_an_invalid_argument():
    with pytest.raises(kv.KvError) as ei:
        kv.memory_location_label(99, 0)
    assert ei.value.code == kv.INVALID_ARGUMENT


def test_decode_remote_layout_of_one_region(goldens):
    """The reference's CUDA pool: one region, item length = page size
    (cuda_backend.rs:304-309), pointers = the region bases."""
    g = goldens["cuda_backend_page_round_trip"]
    mem = kv.TransferableKvCacheMemory([(0x7F0000000000, g["region_byte_len"], g["page_size_bytes"])],
                                       g["page_size_bytes"], kv.LOCATION_ROCM, 0)
    remote = mem.mooncake_decode_remote_layout(g["decode_remote_layout_indices"])
    assert remote.dst_kv_item_len == g["dst_kv_item_len"]
    assert remote.dst_kv_ptrs == [0x7F0000000000]
    assert remote.dst_kv_indices == g["decode_remote_layout_indices"]


def test_decode_remote_layout_splits_the_page_over_regions():
    """page_size_bytes / regions().len() (transfer.rs:1701): two regions of a
    256-byte logical page advertise items of 128 bytes; the integer division
    of the reference is kept for three regions."""
    two = kv.TransferableKvCacheMemory([(0x1000, 4096, 128), (0x9000, 4096, 128)], 256, kv.LOCATION_CPU, 0)
    r = two.mooncake_decode_remote_layout([4, 5])
    assert r.dst_kv_ptrs == [0x1000, 0x9000] and r.dst_kv_item_len == 128
    three = kv.TransferableKvCacheMemory([(0x1000, 100, 100)] * 3, 256, kv.LOCATION_CPU, 0)
    assert three.mooncake_decode_remote_layout([0]).dst_kv_item_len == 256 // 3


def test_decode_remote_layout_needs_a_region():
    empty = kv.TransferableKvCacheMemory([], 256, kv.LOCATION_ROCM, 0)
    with pytest.raises(kv.KvError) as ei:
        empty.mooncake_decode_remote_layout([0])
    assert ei.value.variant == "Descriptor"


def test_storage_entry_points_reject_null_without_a_gpu():
    lib = kv.lib()
    assert lib.sgl_rocm_kv_storage_destroy(None) == kv.OK
    assert lib.sgl_rocm_kv_slot_map_destroy(None) == kv.OK
    assert lib.sgl_rocm_kv_storage_byte_len(None) == 0
    assert lib.sgl_rocm_kv_storage_page_size_bytes(None) == 0
    assert lib.sgl_rocm_kv_storage_device(None) == -1
    assert lib.sgl_rocm_kv_slot_map_len(None) == 0
    out = ctypes.c_void_p()
    assert lib.sgl_rocm_kv_storage_allocate(None, 64, 64, ctypes.byref(out)) == kv.INVALID_ARGUMENT
    assert out.value is None
    assert lib.sgl_rocm_kv_storage_clear(None) == kv.INVALID_ARGUMENT
    assert lib.sgl_rocm_kv_storage_validate_layout(None, None) == kv.INVALID_ARGUMENT
    assert lib.sgl_rocm_kv_memory_info(None, None, None) == kv.INVALID_ARGUMENT
    assert lib.sgl_rocm_kv_storage_allocate_placed(None, 64, 64, None, None, None, 3, None,
                                                   ctypes.byref(out), None) == kv.INVALID_ARGUMENT
    assert out.value is None


def test_placement_report_matches_the_header():
    """sgl_kv_placement_report: two u32, a u64 and SGL_KV_PLACEMENT_MAX_CANDIDATES floats."""
    assert kv.PLACEMENT_MAX_CANDIDATES == 8
    assert ctypes.sizeof(kv._PlacementReport) == 4 + 4 + 8 + 4 * 8


def test_storage_status_names():
    for code, name in [(kv.STORAGE_SIZE_MISMATCH, "StorageSizeMismatch"),
                       (kv.STORAGE_SLOT_MAP_CAPACITY_MISMATCH, "SlotMapCapacityMismatch"),
                       (kv.STORAGE_PAGE_BUFFER_SIZE_MISMATCH, "PageBufferSizeMismatch"),
                       (kv.STORAGE_SIZE_OVERFLOW, "SizeOverflow"),
                       (kv.ZERO_ALLOCATION, "ZeroAllocation"),
                       (kv.UNSUPPORTED_MEMORY_LOCATION, "UnsupportedMemoryLocation"),
                       (kv.STORAGE_DESCRIPTOR, "Descriptor")]:
        assert kv.status_name(code) == name
