"""GPU tests of the batched tensor-slot copies (sgl_rocm_kv_write_tensor_slots
/ _read_tensor_slots, and sgl_rocm_kv_write_tensor_pair_slots for both
tensors of a layer): the reference writes MLA cache rows one token and one
tensor at a time with CudaKvStorage::write_tensor_slot_from_device
(crates/sglang-srt/src/cuda_kv_cache.rs:258-294, called from
cuda_mla.rs:256-271); here a whole batch of tokens is one launch.

The expected pool bytes come from the CPU oracle (oracle/kv_oracle.c): its
row-granular unpack and pack over a one-tensor pool whose geometry comes from
the oracle's own pair layout arithmetic (ora_pair_tensor_token_byte_range,
pinned by the reference's asymmetric-pair goldens); nothing expected here is
computed by the product's PagedKvCacheLayout.
"""
import numpy as np
import pytest

import oracle
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


class _OraclePair:
    """The oracle's description of a tensor-pair pool: L layers, page size P,
    `pages` pages, key and value widths kb, vb bytes per token per layer."""

    def __init__(self, layers, P, pages, kb, vb):
        self.kb, self.vb = kb, vb
        bpt = layers * (kb + vb)
        self.layout = oracle.layout(P, layers, 2, bpt, P * bpt, pages)

    def width(self, tensor):
        return self.kb if tensor == 0 else self.vb

    def tensor_pool(self, layer, tensor):
        """One tensor of one layer as a one-tensor oracle pool."""
        rc, rng = oracle.pair_tensor_token_byte_range(self.layout, self.kb, self.vb, 0, layer, tensor, 0)
        assert rc == 0
        lay = self.layout
        return oracle.Pool(lay.page_size, lay.page_size_bytes, lay.page_count, (rng[0],),
                           self.width(tensor), 1, 1, False)

    def slot_range(self, layer, tensor, slot):
        P = self.layout.page_size
        rc, rng = oracle.pair_tensor_token_byte_range(self.layout, self.kb, self.vb, int(slot) // P, layer,
                                                      tensor, int(slot) % P)
        assert rc == 0
        return rng


def _opair(layers, page_size, pages, key=576, value=512):
    return _OraclePair(layers, page_size, pages, key * 2, value * 2)


def _expected(o, pool_h, layer, tensor, slots, rows, stride):
    """The pool after writing rows[i * stride ..] to slot slots[i] of
    (layer, tensor), by the oracle's unpack."""
    want = pool_h.copy()
    oracle.unpack(o.tensor_pool(layer, tensor), want, np.asarray(slots, np.uint64),
                  np.ascontiguousarray(rows), None, stride)
    return want


def _expected_rows(o, pool_h, layer, tensor, slots, stride, fill=0):
    """The rows a read of (layer, tensor) at `slots` must produce, by the
    oracle's pack."""
    n = len(slots)
    rows = np.full(n * stride, fill, np.uint8)
    oracle.pack(o.tensor_pool(layer, tensor), pool_h, np.asarray(slots, np.uint64), rows, None, stride)
    return rows


@pytest.mark.parametrize("page_size,count,pad", [(64, 1, 0), (64, 3000, 0), (1, 777, 48),
                                                 (16, 4096, 8)])
def test_mla_pair_write_then_read(k, page_size, count, pad):
    """Key (1,152 B) and value (1,024 B) rows of one layer written for a
    batch of slots, then read back; unequal widths, one call per tensor."""
    layers, pages = 3, max(64, -(-2 * count // page_size))
    lay = _mla_layout(layers, page_size, pages)
    o = _opair(layers, page_size, pages)
    print(f"[gpu] MLA tensor slots P={page_size} count={count} pad={pad}", flush=True)
    rng = np.random.default_rng(count + page_size)
    pool_h = rng.integers(0, 256, lay.total_byte_len, dtype=np.uint8)
    pool = hip.DeviceBuffer.from_array(pool_h)
    slots_h = rng.choice(pages * page_size, size=count, replace=False).astype(np.uint64)
    slots = hip.DeviceBuffer.from_array(slots_h)
    want = pool_h
    for tensor in (0, 1):
        stride = o.width(tensor) + pad
        rows_h = rng.integers(0, 256, count * stride, dtype=np.uint8)
        src = hip.DeviceBuffer.from_array(rows_h)
        k.write_tensor_slots(lay, _db(pool), 1, tensor, _db(slots), count, _db(src),
                             source_row_stride=stride)
        want = _expected(o, want, 1, tensor, slots_h, rows_h, stride)
        back = hip.DeviceBuffer(count * stride)
        back.upload(np.zeros(count * stride, np.uint8))
        k.read_tensor_slots(lay, _db(pool), 1, tensor, _db(slots), count, _db(back),
                            destination_row_stride=stride)
        k.check_errors()
        np.testing.assert_array_equal(back.download(), _expected_rows(o, want, 1, tensor, slots_h, stride))
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
    o = _opair(2, 16, 8)
    pool_h = np.random.default_rng(1).integers(0, 256, lay.total_byte_len, dtype=np.uint8)
    pool = hip.DeviceBuffer.from_array(pool_h)
    slots_h = np.array([3, 16 * 8, 5], np.uint64)
    slots = hip.DeviceBuffer.from_array(slots_h)
    rows_h = np.full(3 * 1152, 7, np.uint8)
    src = hip.DeviceBuffer.from_array(rows_h)
    k.write_tensor_slots(lay, _db(pool), 0, 0, _db(slots), 3, _db(src))
    with pytest.raises(kv.KvError) as e:
        k.check_errors()
    assert e.value.variant == "DeviceSlotIndexOutOfRange"
    want = pool_h.copy()
    for s in (3, 5):
        a, b = o.slot_range(0, 0, s)
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
    o = _opair(layers, page_size, pages)
    print(f"[gpu] MLA pair slots P={page_size} count={count} pads={pads} offsets={offsets}", flush=True)
    rng = np.random.default_rng(count + 3 * page_size)
    pool_h = rng.integers(0, 256, lay.total_byte_len, dtype=np.uint8)
    slots_h = rng.choice(pages * page_size, size=count, replace=False).astype(np.uint64)
    slots = hip.DeviceBuffer.from_array(slots_h)
    rows, strides, want = [], [], pool_h
    for t in (0, 1):
        strides.append(o.width(t) + pads[t])
        rows.append(rng.integers(0, 256, offsets[t] + count * strides[t], dtype=np.uint8))
        want = _expected(o, want, 2, t, slots_h, rows[t][offsets[t]:], strides[t])
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
    slots_h = np.array([3, 16 * 8, 5], np.uint64)
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
    o = _opair(2, 16, 8)
    want = pool_h.copy()
    for s in (3, 5):
        a, b = o.slot_range(1, 0, s)
        want[a:b] = 7
        a, b = o.slot_range(1, 1, s)
        want[a:b] = 9
    np.testing.assert_array_equal(pool.download(), want)


@pytest.mark.parametrize("seed", range(10))
def test_random_pair_shapes(k, seed):
    """Random key and value widths (unequal, odd or 16-byte multiples),
    layers, page sizes, strides and batch sizes: the one-launch pair write,
    the per-tensor writes and the per-tensor reads, against the oracle."""
    rng = np.random.default_rng(500 + seed)
    layers, P = int(rng.integers(1, 5)), int(rng.choice([1, 2, 16, 64]))
    elt = int(rng.choice([1, 2]))
    kd, vd = int(rng.integers(1, 700)), int(rng.integers(1, 600))
    if rng.random() < 0.5:   # widths whose bytes are whole 16-byte vectors
        kd, vd = kd // 16 * 16 + 16, vd // 16 * 16 + 16
    count = int(rng.choice([1, 5, 64, 333, 1000]))
    pages = -(-count // P) + int(rng.integers(1, 4))
    kb, vb = kd * elt, vd * elt
    model = kv.KvCacheModelLayout.tensor_pair(layers, 1, kd, 1, vd)
    lay = kv.PagedKvCacheLayout.for_model(model, "bf16" if elt == 2 else "fp8_e4m3", P, P * pages)
    o = _OraclePair(layers, P, pages, kb, vb)
    layer = int(rng.integers(0, layers))
    print(f"[gpu] random pair slots {seed}: L={layers} P={P} key={kb} B value={vb} B count={count}",
          flush=True)
    pool_h = rng.integers(0, 256, lay.total_byte_len, dtype=np.uint8)
    slots_h = rng.choice(pages * P, size=count, replace=False).astype(np.uint64)
    slots = hip.DeviceBuffer.from_array(slots_h)
    strides = [kb + int(rng.choice([0, 0, 1, 16])), vb + int(rng.choice([0, 0, 3, 32]))]
    rows = [rng.integers(0, 256, count * st, dtype=np.uint8) for st in strides]
    want = pool_h
    for t in (0, 1):
        want = _expected(o, want, layer, t, slots_h, rows[t], strides[t])
    keys, values = (hip.DeviceBuffer.from_array(r) for r in rows)
    pool = hip.DeviceBuffer.from_array(pool_h)
    k.write_tensor_pair_slots(lay, _db(pool), layer, _db(slots), count, _db(keys), _db(values),
                              keys_row_stride=strides[0], values_row_stride=strides[1])
    k.check_errors()
    np.testing.assert_array_equal(pool.download(), want)
    pool2 = hip.DeviceBuffer.from_array(pool_h)
    for t, buf in ((0, keys), (1, values)):
        k.write_tensor_slots(lay, _db(pool2), layer, t, _db(slots), count, _db(buf),
                             source_row_stride=strides[t])
    k.check_errors()
    np.testing.assert_array_equal(pool2.download(), want)
    for t in (0, 1):
        back = hip.DeviceBuffer(count * strides[t])
        back.upload(np.full(count * strides[t], 0xC3, np.uint8))
        k.read_tensor_slots(lay, _db(pool), layer, t, _db(slots), count, _db(back),
                            destination_row_stride=strides[t])
        k.check_errors()
        np.testing.assert_array_equal(back.download(),
                                      _expected_rows(o, want, layer, t, slots_h, strides[t], fill=0xC3))
