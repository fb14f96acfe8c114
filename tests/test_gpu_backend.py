"""GPU tests of the transfer backend (sgl_rocm_kv_backend_*), the device
counterpart of KvTransferBackend (crates/sglang-srt/src/transfer.rs:
1145-1151), and of the multi-layer pool-to-pool launch it uses.

Every moved byte is checked against the CPU oracle (oracle/kv_oracle.c) on
the same seeded pools, bit for bit: the prefill pool is page size 1 NHD, the
decode pool page size 16 HND with its own page table, and spans carry cached
prefixes (token_offset > 0, as in crates/sglang-srt/tests/pd_transfer_plan.rs:
85-114). Event semantics follow the Mooncake executor's poll and cancel
(transfer.rs:2605-2674): each finished span is reported once with its
bootstrap room and descriptor checksum; a canceled room reports nothing.
"""
import numpy as np
import pytest

import oracle
import sgl_rocm_kv as kv
from sgl_rocm_kv import hip
from sgl_rocm_kv import workloads as wl

pytestmark = pytest.mark.gpu

L, H, D = 4, 8, 128          # layers, KV heads, head dim (bf16): 2 KiB rows
P_PREFILL, P_DECODE = 1, 16
PREFILL_PAGES, DECODE_PAGES = 4096, 256


def _say(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def k():
    if hip.device_count() == 0:
        pytest.fail("no GPU visible: the gpu tests need an MI355X")
    ctx = kv.RocmKvPairCopyKernels(0)
    yield ctx
    ctx.close()


def _layouts(p_prefill=P_PREFILL):
    """The prefill pool holds PREFILL_PAGES * P_PREFILL slots at any page size."""
    pre = kv.PagedKvCacheLayout.new(kv.KvCacheRuntimeLayout.for_model("bf16", p_prefill, L, H, D),
                                    PREFILL_PAGES * P_PREFILL // p_prefill)
    dec = kv.PagedKvCacheLayout.new(kv.KvCacheRuntimeLayout.for_model("bf16", P_DECODE, L, H, D),
                                    DECODE_PAGES)
    return pre, dec


def _opool(view: kv.PoolView) -> oracle.Pool:
    t = view.tensor_count
    return oracle.Pool(view.page_size, view.page_stride_bytes, view.page_count,
                       tuple(view.tensor_offset[:t]), view.row_bytes, t, view.heads,
                       view.head_layout == kv.HND)


class _Pools:
    """Seeded prefill and decode pools on the device, with host copies of
    what the decode pool must hold after the submitted spans."""

    def __init__(self, seed, p_prefill=P_PREFILL):
        self.pre, self.dec = _layouts(p_prefill)
        rng = np.random.default_rng(seed)
        self.src_h = rng.integers(0, 256, self.pre.total_byte_len, dtype=np.uint8)
        self.dst_h = rng.integers(0, 256, self.dec.total_byte_len, dtype=np.uint8)
        self.src = hip.DeviceBuffer.from_array(self.src_h)
        self.dst = hip.DeviceBuffer.from_array(self.dst_h)
        self.want = self.dst_h.copy()

    def register(self, backend):
        backend.register(self.pre, self.src.ptr, self.src.nbytes, self.dec, self.dst.ptr,
                         self.dst.nbytes, decode_head_layout=kv.HND)

    def expect(self, token_offset, cache_slots, page_table):
        """Applies one span to the expected decode pool with the oracle."""
        tokens = token_offset + np.arange(len(cache_slots), dtype=np.uint64)
        table = np.asarray(page_table, dtype=np.uint64)
        dst_slots = table[tokens // P_DECODE] * P_DECODE + tokens % P_DECODE
        for layer in range(L):
            sv = self.pre.pool_view(self.src.ptr, self.src.nbytes, layer, kv.NHD, H)
            dv = self.dec.pool_view(self.dst.ptr, self.dst.nbytes, layer, kv.HND, H)
            oracle.transfer(_opool(sv), self.src_h, cache_slots, _opool(dv), self.want, dst_slots,
                            threads=4)

    def check(self):
        np.testing.assert_array_equal(self.dst.download(), self.want)


def _span(rng, token_offset, count, pages):
    """A request's prefill slots (distinct, shuffled pages of size 1) and a
    decode page table covering tokens 0 .. token_offset+count."""
    slots = rng.choice(PREFILL_PAGES, size=count, replace=False).astype(np.uint64)
    need = -(-(token_offset + count) // P_DECODE)
    table = rng.choice(pages, size=need, replace=False).astype(np.int32)
    return slots, table


def _checksum(room, token_offset, slots):
    pages = [int(s) for s in slots]
    return kv.transfer_span_checksum(f"req-{room}", "10.0.0.8", 8200, room, 0, token_offset,
                                     len(slots), P_PREFILL, pages,
                                     [p for p in pages])


@pytest.mark.parametrize("mode", [kv.BACKEND_DIRECT, kv.BACKEND_STAGED])
def test_backend_spans_match_oracle(k, mode):
    """Spans with and without cached prefixes, a no-op span, and in-order
    completion events carrying each span's room and checksum."""
    name = "direct" if mode == kv.BACKEND_DIRECT else "staged"
    _say(f"backend {name}: 4 spans over {L} layers")
    rng = np.random.default_rng(100 + mode)
    pools = _Pools(seed=7 + mode)
    b = kv.RocmKvTransferBackend(k, mode, max_rows=512)
    pools.register(b)
    # Each request owns a disjoint group of decode pages.
    groups = rng.permutation(DECODE_PAGES).reshape(8, -1)
    cases = [(11, 0, 37), (12, 16, 50), (13, 5, 0), (14, 32, 300)]
    sums = {}
    for i, (room, off, n) in enumerate(cases):
        slots, table = _span(rng, off, n, groups[i])
        sums[room] = _checksum(room, off, slots)
        b.submit(room, sums[room], off, slots, table)
        if n:
            pools.expect(off, slots, table)
    b.wait()
    events, pending = b.poll()
    assert pending == 0
    assert [e.bootstrap_room for e in events] == [c[0] for c in cases]
    for e in events:
        assert e.status == kv.TRANSFER_COMPLETED and e.error_code == 0
        assert e.descriptor_checksum == sums[e.bootstrap_room]
    assert b.poll() == ([], 0)  # each span is reported once
    pools.check()
    b.close()


def test_backend_poll_capacity_and_cancel(k):
    """poll returns at most `capacity` events and keeps the rest; a canceled
    room never reports; pending counts spans not yet reported."""
    rng = np.random.default_rng(5)
    pools = _Pools(seed=8)
    b = kv.RocmKvTransferBackend(k, kv.BACKEND_DIRECT, max_rows=256)
    pools.register(b)
    groups = rng.permutation(DECODE_PAGES).reshape(8, -1)
    for i, room in enumerate((21, 22, 23, 24)):
        slots, table = _span(rng, 0, 100, groups[i])
        b.submit(room, f"{room:064x}", 0, slots, table)
        pools.expect(0, slots, table)
    b.cancel(23)
    b.wait()
    first, pending = b.poll(capacity=1)
    assert [e.bootstrap_room for e in first] == [21] and pending == 2
    rest, pending = b.poll()
    assert [e.bootstrap_room for e in rest] == [22, 24] and pending == 0
    assert rest[0].descriptor_checksum == f"{22:064x}"
    # A canceled span's device work still ran to completion.
    pools.check()
    b.shutdown()
    # After shutdown the backend can be registered again.
    pools.register(b)
    b.close()


def test_backend_spans_in_flight_limit(k):
    """Each span in flight holds one of the backend's 1,024 error words. The
    1,025th unpolled span is refused on the host with a typed error and
    nothing is enqueued for it; once poll has reported the finished spans,
    their words are free and a new span moves and completes."""
    rng = np.random.default_rng(6)
    pools = _Pools(seed=9)
    b = kv.RocmKvTransferBackend(k, kv.BACKEND_DIRECT, max_rows=16)
    pools.register(b)
    pages = rng.permutation(DECODE_PAGES)
    _say("backend: 1,024 one-token spans in flight, then one more")
    for i in range(1024):
        table = [int(pages[i % DECODE_PAGES])]
        slot = np.array([rng.integers(0, PREFILL_PAGES)], dtype=np.uint64)
        b.submit(1000 + i, f"{i:064x}", i % P_DECODE, slot, table)
        pools.expect(i % P_DECODE, slot, table)
    with pytest.raises(kv.KvError) as e:
        b.submit(5000, "0" * 64, 0, np.array([1], dtype=np.uint64), [0])
    assert e.value.variant == "DimensionTooLarge" and e.value.name == "spans in flight"
    b.wait()
    events, pending = [], 1
    while pending:
        got, pending = b.poll(capacity=300)
        events += got
    assert [e.bootstrap_room for e in events] == [1000 + i for i in range(1024)]
    assert all(e.status == kv.TRANSFER_COMPLETED for e in events)
    slot = np.array([7], dtype=np.uint64)
    table = [int(pages[-1])]
    b.submit(5001, "1" * 64, 3, slot, table)
    pools.expect(3, slot, table)
    b.wait()
    [done], pending = b.poll()
    assert done.bootstrap_room == 5001 and done.status == kv.TRANSFER_COMPLETED and pending == 0
    pools.check()
    b.close()


def test_backend_staged_spans_reuse_staging_in_order(k):
    """Staged spans share one set of staging buffers: many back-to-back
    submissions must each complete intact."""
    rng = np.random.default_rng(9)
    pools = _Pools(seed=10)
    b = kv.RocmKvTransferBackend(k, kv.BACKEND_STAGED, max_rows=128)
    pools.register(b)
    groups = rng.permutation(DECODE_PAGES).reshape(16, -1)
    rooms = list(range(31, 47))
    for i, room in enumerate(rooms):
        off = int(rng.integers(0, 32))
        n = int(rng.integers(1, 129))
        n = min(n, (len(groups[i]) * P_DECODE) - off)
        slots, table = _span(rng, off, n, groups[i])
        b.submit(room, "", off, slots, table)
        pools.expect(off, slots, table)
    seen = []
    for _ in range(2 * len(rooms)):
        if len(seen) == len(rooms):
            break
        events, pending = b.poll(capacity=3)
        seen += [e.bootstrap_room for e in events]
        assert pending == len(rooms) - len(seen)
        if not events:
            b.wait()
    assert seen == rooms
    pools.check()
    b.close()


def test_backend_submit_validation(k):
    """Bad spans are refused on the host before anything is enqueued, with
    the reference's layout error variants; nothing is written."""
    rng = np.random.default_rng(3)
    pools = _Pools(seed=11)
    b = kv.RocmKvTransferBackend(k, kv.BACKEND_DIRECT, max_rows=64)
    with pytest.raises(kv.KvError) as e:          # nothing registered yet
        b.submit(1, "", 0, [0], [0])
    assert e.value.code == 12
    pools.register(b)
    with pytest.raises(kv.KvError) as e:          # registered twice
        pools.register(b)
    assert e.value.code == 12
    slots, table = _span(rng, 0, 40, np.arange(DECODE_PAGES))
    bad = slots.copy()
    bad[7] = PREFILL_PAGES                        # past the prefill pool
    with pytest.raises(kv.KvError) as e:
        b.submit(2, "", 0, bad, table)
    assert e.value.variant == "BatchSlotOutOfRange" and e.value.fields[:3] == (7, PREFILL_PAGES,
                                                                                PREFILL_PAGES)
    with pytest.raises(kv.KvError) as e:          # page table too short
        b.submit(3, "", 0, slots, table[:2])
    assert e.value.code == 12 and e.value.name == "dst_page_table"
    neg = table.copy()
    neg[1] = -1
    with pytest.raises(kv.KvError) as e:
        b.submit(4, "", 0, slots, neg)
    assert e.value.variant == "PageOutOfRange"
    past = table.copy()
    past[2] = DECODE_PAGES
    with pytest.raises(kv.KvError) as e:
        b.submit(5, "", 0, slots, past)
    assert e.value.variant == "PageOutOfRange" and e.value.fields[:2] == (DECODE_PAGES,
                                                                          DECODE_PAGES)
    big, big_table = _span(rng, 0, 65, np.arange(DECODE_PAGES))
    with pytest.raises(kv.KvError) as e:          # more rows than max_rows
        b.submit(6, "", 0, big, big_table)
    assert e.value.code == 3
    assert b.poll() == ([], 0)
    pools.check()                                 # untouched
    b.close()


def test_backend_register_rejects_mismatched_pools(k):
    pre = kv.PagedKvCacheLayout.new(kv.KvCacheRuntimeLayout.for_model("bf16", 1, L, H, D), 64)
    other = kv.PagedKvCacheLayout.new(kv.KvCacheRuntimeLayout.for_model("bf16", 16, L + 1, H, D), 4)
    a, c = hip.DeviceBuffer(pre.total_byte_len), hip.DeviceBuffer(other.total_byte_len)
    b = kv.RocmKvTransferBackend(k, kv.BACKEND_DIRECT, max_rows=16)
    with pytest.raises(kv.KvError) as e:
        b.register(pre, a.ptr, a.nbytes, other, c.ptr, c.nbytes)
    assert e.value.code == 12
    with pytest.raises(kv.KvError) as e:          # decode allocation too small
        b.register(pre, a.ptr, a.nbytes, pre, c.ptr, pre.total_byte_len - 1)
    assert e.value.code == 11 and e.value.name == "decode"
    assert e.value.fields[1:] == (pre.total_byte_len, pre.total_byte_len - 1)
    b.register(pre, a.ptr, a.nbytes, pre, c.ptr, pre.total_byte_len)  # exactly enough
    b.close()


def test_transfer_layers_matches_per_layer_oracle(k):
    """One pool-to-pool launch over all layers (P=1 NHD -> P=64 HND) equals
    the per-layer oracle; a layer span that runs past the destination is
    refused on the host."""
    t = wl.scaled(wl.c2(), 3000, seed=6)
    t.dst = wl.PoolSpec(64, t.dst.page_count, kv.HND)
    sh = t.shape
    layers = 6
    _say(f"transfer_layers {t.name}: {t.rows} rows x {layers} layers")
    rng = np.random.default_rng(22)
    src_h = rng.integers(0, 256, t.src.byte_len(sh), dtype=np.uint8)
    dst_h = rng.integers(0, 256, t.dst.byte_len(sh), dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer.from_array(dst_h)
    ss, ds = hip.DeviceBuffer.from_array(t.src_slots), hip.DeviceBuffer.from_array(t.dst_slots)

    def view(buf, spec, layer):
        return kv.pool_view(buf.ptr, buf.nbytes, page_size=spec.page_size,
                            page_stride_bytes=spec.page_stride(sh), page_count=spec.page_count,
                            tensor_offset=spec.tensor_offsets(sh, layer), row_bytes=sh.row_bytes,
                            tensor_count=sh.tensors, heads=sh.heads, head_layout=spec.head_layout)

    def opool(spec, layer):
        return oracle.Pool(spec.page_size, spec.page_stride(sh), spec.page_count,
                           spec.tensor_offsets(sh, layer), sh.row_bytes, sh.tensors, sh.heads,
                           spec.head_layout == kv.HND)

    first = 3
    s_stride = t.src.tensor_offsets(sh, first + 1)[0] - t.src.tensor_offsets(sh, first)[0]
    d_stride = t.dst.tensor_offsets(sh, first + 1)[0] - t.dst.tensor_offsets(sh, first)[0]
    k.transfer_layers(view(src, t.src, first), s_stride, layers, kv.device_buffer(ss.ptr, ss.nbytes),
                      t.rows, view(dst, t.dst, first), d_stride,
                      kv.device_buffer(ds.ptr, ds.nbytes))
    k.check_errors()
    for layer in range(first, first + layers):
        oracle.transfer(opool(t.src, layer), src_h, t.src_slots, opool(t.dst, layer), dst_h,
                        t.dst_slots, threads=4)
    np.testing.assert_array_equal(dst.download(), dst_h)
    with pytest.raises(kv.KvError):
        k.transfer_layers(view(src, t.src, first), s_stride, sh.layers,
                          kv.device_buffer(ss.ptr, ss.nbytes), t.rows, view(dst, t.dst, first),
                          d_stride, kv.device_buffer(ds.ptr, ds.nbytes))


@pytest.mark.parametrize("mode", [kv.BACKEND_DIRECT, kv.BACKEND_STAGED])
def test_bootstrap_frames_drive_the_backend(k, mode):
    """The decode side advertises its pool in bootstrap frames: KVArgs with
    dst_kv_ptrs = [pool base] and the decode-layout extension (page size 16,
    head-major), then one transfer frame per request carrying its page
    table as dst_kv_indices and decode_prefix_len. The prefill side
    ingests the frames, rebuilds the decode registration from the
    advertised layout and base pointer, and moves each request's uncached
    tokens through the backend; every byte matches the oracle."""
    rng = np.random.default_rng(300 + mode)
    pools = _Pools(seed=30 + mode)
    decode_layout = kv.DecodeLayout(pools.dec, kv.HND, H)
    frames = [kv.encode_kv_args_frame(endpoint="10.0.0.9", dst_port=41001, mooncake_session_id="decode-0",
                                      dst_kv_ptrs=[pools.dst.ptr],
                                      dst_kv_item_len=pools.dec._c.runtime.page_size_bytes,
                                      decode_layout=decode_layout)]
    groups = rng.permutation(DECODE_PAGES).reshape(8, -1)
    requests = {}
    for i, (room, cached, n) in enumerate([(51, 0, 90), (52, 32, 140), (53, 16, 1)]):
        slots, table = _span(rng, cached, n, groups[i])
        requests[room] = (cached, slots)
        frames.append(kv.encode_transfer_frame(room=room, endpoint="10.0.0.9", dst_port=41001,
                                               mooncake_session_id="decode-0", dst_kv_indices=table,
                                               dst_aux_index=0, decode_prefix_len=cached + n))
    state = kv.PrefillBootstrapState()
    for f in frames:
        state.ingest_mooncake_bootstrap_frame(f)
    b = kv.RocmKvTransferBackend(k, mode, max_rows=256)
    registered = False
    for room, (cached, slots) in requests.items():
        assert state.transfer_status(room) == "WaitingForInput"
        [(session, remote)] = state.remote_kv_layouts_for_room(room)
        adv = remote["decode_layout"]
        assert session == "decode-0" and adv is not None and adv.head_layout == kv.HND
        if not registered:
            base = remote["dst_kv_ptrs"][0]
            b.register(pools.pre, pools.src.ptr, pools.src.nbytes, adv.layout, base,
                       adv.layout.total_byte_len, decode_head_layout=adv.head_layout,
                       decode_heads=adv.heads)
            registered = True
        table = remote["dst_kv_indices"]
        b.submit(room, "", cached, slots, table)
        pools.expect(cached, slots, table)
    b.wait()
    events, pending = b.poll()
    assert pending == 0 and sorted(e.bootstrap_room for e in events) == sorted(requests)
    assert all(e.status == kv.TRANSFER_COMPLETED for e in events)
    pools.check()
    b.close()
    state.close()


@pytest.mark.parametrize("mode", [kv.BACKEND_DIRECT, kv.BACKEND_STAGED])
def test_prefill_batch_plan_drives_the_backend(k, mode):
    """The scheduler's route to the backend: prompts are matched against the
    prefill side's token-prefix cache (RadixCache::match_prefix_page_aligned,
    cache.rs:532-540), the uncached suffixes get slots from the page
    allocator, the batch's plan (from_prefill_worker_batch_with_page_size,
    transfer.rs:604-668) yields one span per PD request with its cached
    prefix as the token offset, and each span goes to the backend under its
    own decode page table. Requests without disaggregated params get no span
    but still own slots in the batch. Every decode-pool byte matches the
    oracle, and each event carries the checksum of its span's fields."""
    rng = np.random.default_rng(400 + mode)
    pools = _Pools(seed=40 + mode)
    alloc = kv.CachePageAllocator(PREFILL_PAGES * P_PREFILL, P_PREFILL)
    cache = kv.RadixCache()
    # Two cached prompts: 48 and 21 tokens already in the prefill pool.
    shared_a = [int(t) for t in rng.integers(0, 1000, 48)]
    shared_b = [int(t) for t in rng.integers(1000, 2000, 21)]
    for toks in (shared_a, shared_b):
        cache.insert(toks, alloc.allocate(len(toks)))
    prompts = [shared_a + [int(t) for t in rng.integers(0, 5000, 70)],   # 48 cached, 70 move
               [int(t) for t in rng.integers(5000, 6000, 33)],           # nothing cached
               shared_b[:9] + [int(t) for t in rng.integers(0, 5000, 5)],  # 9 cached, no params
               shared_b + [int(t) for t in rng.integers(0, 5000, 200)],  # 21 cached, 200 move
               shared_a[:16]]                                            # fully cached: nothing moves
    has_params = [1, 1, 0, 1, 1]
    cached, inputs, slots = [], [], []
    for p in prompts:
        m = cache.match_prefix_page_aligned(p, P_PREFILL)
        cached.append(m.matched_token_count)
        inputs.append(len(m.remaining_input_ids))
        slots += alloc.allocate(len(m.remaining_input_ids))
    assert cached == [48, 0, 9, 21, 16] and inputs == [70, 33, 5, 200, 0]
    spans = kv.transfer_plan_from_prefill_batch(inputs, cached, has_params, slots, P_PREFILL)
    assert [s.request_index for s in spans] == [0, 1, 3, 4]
    _say(f"batch plan: {len(spans)} spans, {sum(s.token_count for s in spans)} tokens over {L} layers "
         f"({'direct' if mode == kv.BACKEND_DIRECT else 'staged'})")
    b = kv.RocmKvTransferBackend(k, mode, max_rows=256)
    pools.register(b)
    groups = rng.permutation(DECODE_PAGES).reshape(8, -1)
    sums = {}
    for i, s in enumerate(spans):
        room = 60 + s.request_index
        need = -(-(s.token_offset + s.token_count) // P_DECODE)
        table = rng.choice(groups[i], size=need, replace=False).astype(np.int32)
        sums[room] = kv.transfer_span_checksum(f"req-{room}", "10.0.0.8", 8200, room, 0, s.token_offset,
                                               s.token_count, P_PREFILL, s.cache_pages, s.page_indices)
        cache_slots = np.asarray(s.cache_pages, dtype=np.uint64)
        b.submit(room, sums[room], s.token_offset, cache_slots, table)
        if s.token_count:
            pools.expect(s.token_offset, cache_slots, table)
    b.wait()
    events, pending = b.poll()
    assert pending == 0 and [e.bootstrap_room for e in events] == sorted(sums)
    for e in events:
        assert e.status == kv.TRANSFER_COMPLETED and e.descriptor_checksum == sums[e.bootstrap_room]
    pools.check()
    b.close()


@pytest.mark.parametrize("mode", [kv.BACKEND_DIRECT, kv.BACKEND_STAGED])
@pytest.mark.parametrize("p_prefill", [16, 64])
def test_prefill_batch_plan_with_prefill_pages(k, mode, p_prefill):
    """The same route with prefill pages of 16 and 64 tokens, where the
    plan's page rules bite (transfer.rs:679-720): cached prefixes are matched
    page-aligned (match_prefix_page_aligned rounds 50 cached tokens down to
    whole pages), each uncached suffix starts on a fresh page of the
    allocator, so its slots are page-aligned and contiguous within each page,
    and the span's page indices are those pages. A batch whose cached prefix
    is not a whole number of prefill pages (the plain match) is refused with
    UnalignedTokenOffset before anything reaches the backend, and the decode
    pool is unchanged by it. Every decode-pool byte matches the oracle."""
    P = p_prefill
    rng = np.random.default_rng(500 + P + mode)
    pools = _Pools(seed=50 + P + mode, p_prefill=P)
    slots_total = PREFILL_PAGES * P_PREFILL
    alloc = kv.CachePageAllocator(slots_total, P)
    cache = kv.RadixCache()
    shared = [int(t) for t in rng.integers(0, 1000, 2 * P + P // 2 + 3)]   # cached: two pages and a part
    cache.insert(shared, alloc.allocate(len(shared)))
    prompts = [shared + [int(t) for t in rng.integers(0, 5000, 3 * P + 5)],   # two pages cached
               [int(t) for t in rng.integers(5000, 6000, P + 7)],             # nothing cached
               shared[:P + 3] + [int(t) for t in rng.integers(0, 5000, 40)]]  # one page cached
    has_params = [1, 1, 1]
    cached, inputs, slots = [], [], []
    for p in prompts:
        m = cache.match_prefix_page_aligned(p, P)
        cached.append(m.matched_token_count)
        inputs.append(len(m.remaining_input_ids))
        slots += alloc.allocate(len(m.remaining_input_ids))
    assert cached == [2 * P, 0, P]
    spans = kv.transfer_plan_from_prefill_batch(inputs, cached, has_params, slots, P)
    assert [s.token_offset for s in spans] == cached
    for s in spans:   # whole pages of the allocator: the first slot page-aligned, pages contiguous
        pages = np.asarray(s.cache_pages, np.int64)
        assert pages[0] % P == 0 and (np.diff(pages)[np.arange(1, len(pages)) % P != 0] == 1).all()
        assert list(s.page_indices) == sorted(set((pages // P).tolist()), key=list(pages // P).index)
    _say(f"batch plan, prefill pages of {P}: {len(spans)} spans, {sum(s.token_count for s in spans)} tokens "
         f"({'direct' if mode == kv.BACKEND_DIRECT else 'staged'})")
    b = kv.RocmKvTransferBackend(k, mode, max_rows=512)
    pools.register(b)

    # A batch with an unaligned cached prefix (the plain match): refused by the plan.
    m = cache.match_prefix(prompts[0])
    assert m.matched_token_count == len(shared) and m.matched_token_count % P
    bad_slots = alloc.allocate(len(m.remaining_input_ids))
    with pytest.raises(kv.KvError) as ei:
        kv.transfer_plan_from_prefill_batch([len(m.remaining_input_ids)], [m.matched_token_count], [1],
                                            bad_slots, P)
    assert ei.value.variant == "UnalignedTokenOffset"
    assert ei.value.fields == (0, m.matched_token_count, P)
    assert b.poll() == ([], 0)

    groups = rng.permutation(DECODE_PAGES).reshape(8, -1)
    sums = {}
    for i, s in enumerate(spans):
        room = 70 + s.request_index
        need = -(-(s.token_offset + s.token_count) // P_DECODE)
        table = rng.choice(groups[i], size=need, replace=False).astype(np.int32)
        sums[room] = kv.transfer_span_checksum(f"req-{room}", "10.0.0.8", 8200, room, 0, s.token_offset,
                                               s.token_count, P, s.cache_pages, s.page_indices)
        cache_slots = np.asarray(s.cache_pages, dtype=np.uint64)
        b.submit(room, sums[room], s.token_offset, cache_slots, table)
        pools.expect(s.token_offset, cache_slots, table)
    b.wait()
    events, pending = b.poll()
    assert pending == 0 and [e.bootstrap_room for e in events] == sorted(sums)
    for e in events:
        assert e.status == kv.TRANSFER_COMPLETED and e.descriptor_checksum == sums[e.bootstrap_room]
    pools.check()
    b.close()


@pytest.mark.parametrize("mode", [kv.BACKEND_DIRECT, kv.BACKEND_STAGED])
def test_device_table_failure_fails_only_its_span(k, mode):
    """Two spans resolved on the device from device-resident decode page
    tables. One table holds a page past the decode pool: the resolve kernel
    flags that row and skips it (no fault), poll reports that room FAILED
    with DevicePageIndexOutOfRange, its other rows still move, and the other
    span (submitted before and after it) is COMPLETED with every byte moved
    and the neighbouring bytes untouched. Each span owns its error word, so
    the failure is charged to the right room (transfer.rs:2298-2329)."""
    name = "direct" if mode == kv.BACKEND_DIRECT else "staged"
    _say(f"backend {name}: per-span device failure")
    rng = np.random.default_rng(900 + mode)
    pools = _Pools(seed=30 + mode)
    b = kv.RocmKvTransferBackend(k, mode, max_rows=512)
    pools.register(b)
    groups = rng.permutation(DECODE_PAGES).reshape(8, -1)
    good_a = _span(rng, 16, 70, groups[0])
    bad = _span(rng, 0, 90, groups[1])
    good_b = _span(rng, 0, 33, groups[2])
    bad_table = bad[1].copy()
    bad_table[2] = DECODE_PAGES + 3           # tokens 32..47 have no page
    tables = [hip.DeviceBuffer.from_array(t) for t in (good_a[1], bad_table, good_b[1])]
    for room, (slots, _), table, off in ((21, good_a, tables[0], 16), (22, bad, tables[1], 0),
                                         (23, good_b, tables[2], 0)):
        b.submit_device_table(room, f"{room:064x}", off, slots, kv.device_buffer(table.ptr, table.nbytes),
                              table.nbytes // 4)
    pools.expect(16, *good_a)
    pools.expect(0, *good_b)
    # the failed span's rows whose page exists still move
    keep = np.array([i for i in range(90) if i // P_DECODE != 2])
    tok = keep.astype(np.uint64)
    dslots = bad_table[tok // P_DECODE].astype(np.uint64) * P_DECODE + tok % P_DECODE
    for layer in range(L):
        sv = pools.pre.pool_view(pools.src.ptr, pools.src.nbytes, layer, kv.NHD, H)
        dv = pools.dec.pool_view(pools.dst.ptr, pools.dst.nbytes, layer, kv.HND, H)
        oracle.transfer(_opool(sv), pools.src_h, bad[0][keep], _opool(dv), pools.want, dslots)
    b.wait()
    events, pending = b.poll()
    assert pending == 0
    by_room = {e.bootstrap_room: e for e in events}
    assert sorted(by_room) == [21, 22, 23]
    assert by_room[21].status == kv.TRANSFER_COMPLETED and by_room[21].error_code == 0
    assert by_room[23].status == kv.TRANSFER_COMPLETED and by_room[23].error_code == 0
    assert by_room[22].status == kv.TRANSFER_FAILED
    assert kv.status_name(by_room[22].error_code) == "DevicePageIndexOutOfRange"
    pools.check()
    # the words are clean for the next spans: a good span now completes
    again = _span(rng, 0, 20, groups[3])
    t4 = hip.DeviceBuffer.from_array(again[1])
    b.submit_device_table(24, "0" * 64, 0, again[0], kv.device_buffer(t4.ptr, t4.nbytes), len(again[1]))
    pools.expect(0, *again)
    b.wait()
    events, _ = b.poll()
    assert [(e.bootstrap_room, e.status) for e in events] == [(24, kv.TRANSFER_COMPLETED)]
    pools.check()
    b.close()
