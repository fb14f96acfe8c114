"""GPU tests of the batched tensor-slot copies (sgl_rocm_kv_write_tensor_slots
/ _read_tensor_slots, and sgl_rocm_kv_write_tensor_pair_slots for both
tensors of a layer): the reference writes MLA cache rows one token and one
tensor at a time with CudaKvStorage::write_tensor_slot_from_device
(crates/sglang-srt/src/cuda_kv_cache.rs:258-294, called from
cuda_mla.rs:256-271); here a whole batch of tokens is one launch.

The expected pool bytes come from PagedKvCacheLayout::tensor_slot_byte_range
(pinned by the reference's layout goldens), applied on the host in numpy:
for each slot, the token's bytes land at that range and nowhere else.
"""
import numpy as np
import pytest

import sgl_rocm_kv as kv
from sgl_rocm_kv import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def k():
    if hip.device_count() == 0:
        pytest.fail("no GPU visible: the gpu tests need an MI355X")
    ctx = kv.RocmKvPairCopyKernels(0)
    yield ctx
    ctx.close()


def _db(buf):
    return kv.device_buffer(buf.ptr, buf.nbytes)


def _mla_layout(layers, page_size, pages, key=576, value=512):
    """KvCacheModelLayout::tensor_pair(L, 1, key, 1, value) in bf16, as the
    DeepSeek adapter builds it (models/deepseek.rs:360-369)."""
    kb, vb = key * 2, value * 2
    rt = kv.KvCacheRuntimeLayout("bf16", page_size, layers, 1, key, 2, layers * (kb + vb),
                                 layers * (kb + vb) * page_size)
    return kv.PagedKvCacheLayout.new_with_tensor_pair(rt, pages, kb, vb)


def _expected(layout, pool_h, layer, tensor, slots, rows, stride):
    want = pool_h.copy()
    width = layout.tensor_token_bytes(tensor)
    for i, s in enumerate(slots):
        a, b = layout.tensor_slot_byte_range(layer, tensor, int(s))
        assert b - a == width
        want[a:b] = rows[i * stride: i * stride + width]
    return want


@pytest.mark.parametrize("page_size,count,pad", [(64, 1, 0), (64, 3000, 0), (1, 777, 48),
                                                 (16, 4096, 8)])
def test_mla_pair_write_then_read(k, page_size, count, pad):
    """Key (1,152 B) and value (1,024 B) rows of one layer written for a
    batch of slots, then read back; unequal widths, one call per tensor."""
    layers, pages = 3, max(64, -(-2 * count // page_size))
    lay = _mla_layout(layers, page_size, pages)
    print(f"[gpu] MLA tensor slots P={page_size} count={count} pad={pad}", flush=True)
    rng = np.random.default_rng(count + page_size)
    pool_h = rng.integers(0, 256, lay.total_byte_len, dtype=np.uint8)
    pool = hip.DeviceBuffer.from_array(pool_h)
    slots_h = rng.choice(lay.slot_count, size=count, replace=False).astype(np.uint64)
    slots = hip.DeviceBuffer.from_array(slots_h)
    want = pool_h
    for tensor in (0, 1):
        stride = lay.tensor_token_bytes(tensor) + pad
        rows_h = rng.integers(0, 256, count * stride, dtype=np.uint8)
        src = hip.DeviceBuffer.from_array(rows_h)
        k.write_tensor_slots(lay, _db(pool), 1, tensor, _db(slots), count, _db(src),
                             source_row_stride=stride)
        want = _expected(lay, want, 1, tensor, slots_h, rows_h, stride)
        back = hip.DeviceBuffer(count * stride)
        back.upload(np.zeros(count * stride, np.uint8))
        k.read_tensor_slots(lay, _db(pool), 1, tensor, _db(slots), count, _db(back),
                            destination_row_stride=stride)
        k.check_errors()
        got = back.download().reshape(count, stride)[:, :lay.tensor_token_bytes(tensor)]
        np.testing.assert_array_equal(
            got, rows_h.reshape(count, stride)[:, :lay.tensor_token_bytes(tensor)])
    np.testing.assert_array_equal(pool.download(), want)


def test_uniform_layout_offsets_and_host_errors(k, goldens):
    """A uniform K/V layout (the cuda_backend golden: P16, L2, H8, D128):
    writing slot 63 of layer 1, tensor 1 touches exactly bytes
    [522,240, 524,288) (cuda_backend.rs:284-286); bad layer, tensor and
    source ranges are refused on the host."""
    g = goldens["cuda_backend_slot_location"]
    rt = g["runtime"]
    runtime = kv.KvCacheRuntimeLayout(rt["dtype"], rt["page_size"], rt["num_layers"], rt["kv_heads"],
                                      rt["head_dim"], rt["kv_tensors_per_token"],
                                      rt["bytes_per_token"], rt["page_size_bytes"])
    lay = kv.PagedKvCacheLayout.new(runtime, g["page_count"])
    pool_h = np.zeros(lay.total_byte_len, np.uint8)
    pool = hip.DeviceBuffer.from_array(pool_h)
    row = (np.arange(2048) % 251 + 1).astype(np.uint8)
    src = hip.DeviceBuffer.from_array(row)
    slots = hip.DeviceBuffer.from_array(np.array([63], np.uint64))
    k.write_tensor_slots(lay, _db(pool), 1, 1, _db(slots), 1, _db(src))
    k.check_errors()
    got = pool.download()
    loc = g["slot_location_layer_1_tensor_1_slot_63"]
    lo, n = loc["byte_offset"], loc["byte_len"]
    np.testing.assert_array_equal(got[lo:lo + n], row)
    assert not got[:lo].any() and not got[lo + n:].any()
    with pytest.raises(kv.KvError) as e:
        k.write_tensor_slots(lay, _db(pool), 2, 0, _db(slots), 1, _db(src))
    assert e.value.variant == "LayerOutOfRange"
    with pytest.raises(kv.KvError) as e:
        k.write_tensor_slots(lay, _db(pool), 0, 2, _db(slots), 1, _db(src))
    assert e.value.variant == "TensorOutOfRange"
    with pytest.raises(kv.KvError) as e:      # the offset leaves less than one row
        k.write_tensor_slots(lay, _db(pool), 0, 0, _db(slots), 1, _db(src), source_offset=8)
    assert e.value.code == 11
    with pytest.raises(kv.KvError) as e:      # pool allocation shorter than the layout
        k.write_tensor_slots(lay, kv.device_buffer(pool.ptr, lay.total_byte_len - 1), 0, 0,
                             _db(slots), 1, _db(src))
    assert e.value.code == 11


def test_slot_past_pool_is_skipped_and_reported(k):
    lay = _mla_layout(2, 16, 8)
    pool_h = np.random.default_rng(1).integers(0, 256, lay.total_byte_len, dtype=np.uint8)
    pool = hip.DeviceBuffer.from_array(pool_h)
    slots_h = np.array([3, lay.slot_count, 5], np.uint64)
    slots = hip.DeviceBuffer.from_array(slots_h)
    rows_h = np.full(3 * 1152, 7, np.uint8)
    src = hip.DeviceBuffer.from_array(rows_h)
    k.write_tensor_slots(lay, _db(pool), 0, 0, _db(slots), 3, _db(src))
    with pytest.raises(kv.KvError) as e:
        k.check_errors()
    assert e.value.variant == "DeviceSlotIndexOutOfRange"
    want = pool_h.copy()
    for s in (3, 5):
        a, b = lay.tensor_slot_byte_range(0, 0, s)
        want[a:b] = 7
    np.testing.assert_array_equal(pool.download(), want)


@pytest.mark.parametrize("page_size,count,pads,offsets",
                         [(64, 1, (0, 0), (0, 0)), (64, 2500, (0, 0), (0, 0)), (16, 700, (48, 16), (32, 64)),
                          (1, 333, (2, 6), (1, 3))])
def test_mla_pair_in_one_launch(k, page_size, count, pads, offsets):
    """sgl_rocm_kv_write_tensor_pair_slots: a layer's key (1,152 B) and
    value (1,024 B) rows for a batch of slots in one launch, against the
    layout's byte ranges and against the two single-tensor writes. Padded
    strides and offsets that are not multiples of 16 take the byte-wide
    kernel."""
    layers, pages = 3, max(64, -(-2 * count // page_size))
    lay = _mla_layout(layers, page_size, pages)
    print(f"[gpu] MLA pair slots P={page_size} count={count} pads={pads} offsets={offsets}", flush=True)
    rng = np.random.default_rng(count + 3 * page_size)
    pool_h = rng.integers(0, 256, lay.total_byte_len, dtype=np.uint8)
    slots_h = rng.choice(lay.slot_count, size=count, replace=False).astype(np.uint64)
    slots = hip.DeviceBuffer.from_array(slots_h)
    rows, strides, want = [], [], pool_h
    for t in (0, 1):
        strides.append(lay.tensor_token_bytes(t) + pads[t])
        rows.append(rng.integers(0, 256, offsets[t] + count * strides[t], dtype=np.uint8))
        want = _expected(lay, want, 2, t, slots_h, rows[t][offsets[t]:], strides[t])
    keys, values = (hip.DeviceBuffer.from_array(r) for r in rows)
    pool = hip.DeviceBuffer.from_array(pool_h)
    k.write_tensor_pair_slots(lay, _db(pool), 2, _db(slots), count, _db(keys), _db(values),
                              keys_offset=offsets[0], keys_row_stride=strides[0],
                              values_offset=offsets[1], values_row_stride=strides[1])
    k.check_errors()
    got = pool.download()
    np.testing.assert_array_equal(got, want)
    # The same bytes as one write per tensor.
    pool2 = hip.DeviceBuffer.from_array(pool_h)
    for t, buf in ((0, keys), (1, values)):
        k.write_tensor_slots(lay, _db(pool2), 2, t, _db(slots), count, _db(buf), source_offset=offsets[t],
                             source_row_stride=strides[t])
    k.check_errors()
    np.testing.assert_array_equal(pool2.download(), got)


def test_pair_slots_errors(k):
    """Host refusals (layer, one-tensor layout, short stride, short source)
    and a slot past the pool (skipped and reported, the other rows written)."""
    lay = _mla_layout(2, 16, 8)
    pool_h = np.random.default_rng(2).integers(0, 256, lay.total_byte_len, dtype=np.uint8)
    pool = hip.DeviceBuffer.from_array(pool_h)
    slots_h = np.array([3, lay.slot_count, 5], np.uint64)
    slots = hip.DeviceBuffer.from_array(slots_h)
    keys = hip.DeviceBuffer.from_array(np.full(3 * 1152, 7, np.uint8))
    values = hip.DeviceBuffer.from_array(np.full(3 * 1024, 9, np.uint8))
    with pytest.raises(kv.KvError) as e:
        k.write_tensor_pair_slots(lay, _db(pool), 2, _db(slots), 3, _db(keys), _db(values))
    assert e.value.variant == "LayerOutOfRange"
    with pytest.raises(kv.KvError) as e:
        k.write_tensor_pair_slots(lay, _db(pool), 0, _db(slots), 3, _db(keys), _db(values),
                                  values_row_stride=1000)
    assert e.value.code == kv.ROW_STRIDE_TOO_SMALL
    with pytest.raises(kv.KvError) as e:      # the value rows end past their buffer
        k.write_tensor_pair_slots(lay, _db(pool), 0, _db(slots), 3, _db(keys), _db(values), values_offset=16)
    assert e.value.code == 11
    single = kv.PagedKvCacheLayout.new(kv.KvCacheRuntimeLayout("bf16", 16, 2, 1, 576, 1, 2 * 1152, 2 * 1152 * 16), 8)
    with pytest.raises(kv.KvError) as e:
        k.write_tensor_pair_slots(single, _db(pool), 0, _db(slots), 3, _db(keys), _db(values))
    assert e.value.variant == "TensorOutOfRange"
    k.write_tensor_pair_slots(lay, _db(pool), 1, _db(slots), 3, _db(keys), _db(values))
    with pytest.raises(kv.KvError) as e:
        k.check_errors()
    assert e.value.variant == "DeviceSlotIndexOutOfRange"
    want = pool_h.copy()
    for s in (3, 5):
        a, b = lay.tensor_slot_byte_range(1, 0, s)
        want[a:b] = 7
        a, b = lay.tensor_slot_byte_range(1, 1, s)
        want[a:b] = 9
    np.testing.assert_array_equal(pool.download(), want)
