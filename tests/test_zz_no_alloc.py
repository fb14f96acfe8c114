"""The entry point that allocates nothing,
sgl_rocm_kv_paged_attention_async_noalloc, through the C ABI: on two calls in
a row (the second smaller), its outputs equal those of
sgl_rocm_kv_paged_attention_async on the same arguments, bit for bit (same
kernels, same splits; only where the split records live differs), for a GQA
decode and an MLA decode whose sequences are split across workgroups; calls
made back to back on two streams and from two contexts of one device (which
share that device's workspace) are ordered on the device and each still
equals the allocating entry point's result; and a launch whose split records
exceed the static workspace is refused before anything is enqueued.
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


def _layout(P, H, dk, dv, pages):
    kb, vb = H * dk * 2, H * dv * 2
    rt = kv.KvCacheRuntimeLayout("bf16", P, 1, H, dk, 2, kb + vb, (kb + vb) * P)
    if kb == vb:
        return kv.PagedKvCacheLayout.new(rt, pages)
    return kv.PagedKvCacheLayout.new_with_tensor_pair(rt, pages, kb, vb)


class _Decode:
    """A one-layer decode pool with seeded bf16 contents and a batch of
    decode queries; runs either entry point into a fresh output."""

    def __init__(self, rng, P, H, dk, dv, qh, lengths, share=False):
        n = int(max(lengths)) if share else int(sum(lengths))
        pages = -(-n // P) + 2
        self.layout = _layout(P, H, dk, dv, pages)
        pool_h = oracle.f32_to_bf16(rng.standard_normal(self.layout.total_byte_len // 2).astype(np.float32))
        self.pool = hip.DeviceBuffer.from_array(pool_h.view(np.uint8))
        self.qh, self.dk, self.dv = qh, dk, dv
        nq = len(lengths)
        if share:   # every query reads the one request (its own length)
            slots = rng.permutation(self.layout.slot_count)[:max(lengths)].astype(np.uint64)
            rso = np.array([0, len(slots)], np.uint64)
            qri = np.zeros(nq, np.uint32)
        else:
            slots = rng.permutation(self.layout.slot_count)[:n].astype(np.uint64)
            rso = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint64)
            qri = np.arange(nq, dtype=np.uint32)
        q = oracle.f32_to_bf16(rng.standard_normal(nq * qh * dk).astype(np.float32))
        self.plan = kv.PagedAttentionPlan.for_layer(self.layout, 0, nq, len(rso) - 1, len(slots), qh,
                                                    1.0 / np.sqrt(dk), kv.NHD)
        self.bufs = dict(queries=hip.DeviceBuffer.from_array(q),
                         query_request_indices=hip.DeviceBuffer.from_array(qri),
                         query_sequence_lengths=hip.DeviceBuffer.from_array(np.asarray(lengths, np.uint64)),
                         request_slot_offsets=hip.DeviceBuffer.from_array(rso),
                         sequence_slots=hip.DeviceBuffer.from_array(slots), pool=self.pool)
        self.max_len = int(max(lengths))

    def run(self, k, noalloc):
        out = hip.DeviceBuffer(self.plan.output_required_bytes)
        out.fill(0xFF)
        fn = k.paged_attention_async_noalloc if noalloc else k.paged_attention_async
        fn(self.plan, max_sequence_length=self.max_len, output=out, **self.bufs)
        k.check_errors()
        return out.download(dtype=np.uint16)


@pytest.mark.parametrize("shape", ["gqa", "mla"])
def test_noalloc_matches_the_allocating_entry_point_twice(k, shape):
    """Two calls in a row, the second with fewer, shorter queries: each
    no-allocation result equals the allocating entry point's bit for bit."""
    rng = np.random.default_rng(4242 if shape == "gqa" else 4343)
    if shape == "gqa":   # Llama-3-8B decode: 8 KV heads x 128, 32 query heads
        big = _Decode(rng, 64, 8, 128, 128, 32, [3000, 2500, 4096, 17, 900, 3333])
        small = _Decode(rng, 64, 8, 128, 128, 32, [1500, 640])
    else:                # DeepSeek-V3 MLA decode: 1 KV head, keys 576, values 512, 128 heads
        big = _Decode(rng, 64, 1, 576, 512, 128, [5000, 8192, 4000, 777])
        small = _Decode(rng, 64, 1, 576, 512, 128, [2049, 300])
    for case, name in ((big, "first, larger"), (small, "second, smaller")):
        _say(f"noalloc {shape}: {name} call")
        got = case.run(k, noalloc=True)
        want = case.run(k, noalloc=False)
        assert not np.all(want == 0xFFFF)
        np.testing.assert_array_equal(got, want)
    # and the first shape again after the smaller one (the workspace keeps
    # the last call's records; nothing depends on them)
    np.testing.assert_array_equal(big.run(k, noalloc=True), big.run(k, noalloc=False))


def test_noalloc_calls_on_two_streams_and_two_contexts_are_ordered(k):
    """Twelve no-allocation decodes issued back to back, with no host wait,
    alternating between two streams and two contexts of one device, GQA
    (fp32 split records) and MLA (scaled fp16 records) in turn: all of them
    write their records at the start of the one workspace. Each call waits
    on the device for the previous call's combine, so every output equals
    the allocating entry point's, bit for bit."""
    rng = np.random.default_rng(515)
    gqa = _Decode(rng, 64, 8, 128, 128, 32, [4096, 3000, 4096, 2500, 4096, 1234])
    mla = _Decode(rng, 64, 1, 576, 512, 128, [8192, 6000, 8192, 4097])
    want = {id(gqa): gqa.run(k, noalloc=False), id(mla): mla.run(k, noalloc=False)}
    k2 = kv.RocmKvPairCopyKernels(0)
    s1, s2 = hip.Stream(), hip.Stream()
    order = [(gqa, k, s1), (mla, k2, s2), (gqa, k2, s2), (mla, k, s1), (mla, k2, s1), (gqa, k, s2)] * 2
    # every output is allocated and filled before the first launch: a fill
    # on the null stream would otherwise wait for the streams' work
    outs = []
    for case, _, _ in order:
        out = hip.DeviceBuffer(case.plan.output_required_bytes)
        out.fill(0xFF)
        outs.append(out)
    hip.synchronize()
    _say("noalloc: 12 decodes on two streams and two contexts")
    for (case, ctx, s), out in zip(order, outs):
        ctx.paged_attention_async_noalloc(case.plan, max_sequence_length=case.max_len, output=out, stream=s,
                                          **case.bufs)
    s1.synchronize()
    s2.synchronize()
    k.check_errors()
    k2.check_errors()
    for i, ((case, _, _), out) in enumerate(zip(order, outs)):
        np.testing.assert_array_equal(out.download(dtype=np.uint16), want[id(case)], err_msg=f"call {i}")
    s1.destroy()
    s2.destroy()
    k2.close()


def test_noalloc_refuses_records_beyond_the_workspace(k):
    """512 MLA decode queries over one 8,192-token request take two splits
    each (the latent body's 4,096-token slot table): 131,072 scaled-fp16
    split records of 1,040 bytes, 136.3 MB, past the 128 MiB workspace. The
    no-allocation entry point refuses with DimensionTooLarge naming the
    workspace and writes nothing, while the allocating one runs."""
    rng = np.random.default_rng(77)
    case = _Decode(rng, 64, 1, 576, 512, 128, [8192] * 512, share=True)
    out = hip.DeviceBuffer(case.plan.output_required_bytes)
    out.fill(0xAB)
    with pytest.raises(kv.KvError) as ei:
        k.paged_attention_async_noalloc(case.plan, max_sequence_length=8192, output=out, **case.bufs)
    assert ei.value.variant == "DimensionTooLarge" and ei.value.name == "workspace"
    assert ei.value.fields[1] == kv.NOALLOC_WORKSPACE_BYTES and ei.value.fields[0] > kv.NOALLOC_WORKSPACE_BYTES
    k.check_errors()
    assert (out.download() == 0xAB).all()
    k.paged_attention_async(case.plan, max_sequence_length=8192, output=out, **case.bufs)
    k.check_errors()
    assert not (out.download() == 0xAB).all()
