"""GPU tests of the paged-attention reader (sgl_rocm_kv_paged_attention)
against the float64 oracle (oracle.paged_attention, itself pinned against
torch's scaled_dot_product_attention in tests/test_host_attention.py).

Error model and tolerance. The float64 oracle gives out = sum_i w_i v_i
(softmax weights w_i = p_i / l). The kernels compute in fp32 except that
  - the output is rounded to bf16, to nearest even as the reference rounds
    it (cuda_attention.rs:153-155): at most u |out|, u = 2^-8 being bf16's
    unit roundoff (8-bit significand);
  - each weight p_i enters the p.v matrix product as hi + lo, two bf16
    values with |p_i - hi - lo| <= 2^-16 p_i, in every body by default. A
    plan with ATTN_FAST_WEIGHTS lets the MLA latent body (K rows of
    520..576 dims, V rows of 512) round p_i to one bf16 value instead (at
    most u p_i): its matrix cores are the busier unit there.
    The normaliser l sums the unrounded p_i, so a relative error d_i on p_i
    moves the output by sum_i w_i d_i v_i, at most d * sum_i w_i |v_i|;
  - the latent body's split records (when a sequence is split) hold
    y = o / a in fp16 with a = max |o| over the record: y's rounding moves
    a split's o by at most 2^-11 |o| + 2^-25 a, so the output by at most
    2^-11 sum_i w_i |v_i| + 2^-25 max |v| (the second term is below 2.5e-7
    for the values here, |v| < 8, inside the 1e-6 below);
  - the rest is fp32: q.k over at most 576 dims, p.v and l accumulated in
    blocks of 32 over at most 20,000 tokens, exp2 (1 ulp) and the merge of
    split records, together below 2^-12 sum_i w_i |v_i| at these sizes.
So every output element must satisfy
    |got - want| <= u |want| + (2^-12 + [latent] (2^-11 + u [fast])) sum_i w_i |v_i| + 1e-6,
with sum_i w_i |v_i| computed by the oracle for that element: a relative
tolerance of 2^-8 (3.9e-3), the output format's own, plus a term 16 times
smaller outside the latent body. Each case prints its largest |got - want|
and its largest ratio to the bound. A split of a long sequence that is
dropped or counted twice moves the output by far more than the bound (see
test_split_records_are_each_counted_once).

Cases: the reference's own scheduler metadata (causal prefill of two
requests, crates/sglang-srt/tests/cuda_attention.rs:70-97); Llama-3-8B
decode shapes on NHD and HND pages; dims-64 decode shapes (Llama-3.2-1B,
Qwen2-0.5B); a GQA group wider than one workgroup;
MLA widths (576/512, the DeepSeek pair); odd head dims (element-wise
path); long sequences split across workgroups; metadata errors; and an
HND decode pool written by the transfer kernels read back through
attention.
"""
import math
import os

import numpy as np
import pytest

import oracle
import sgl_rocm_kv as kv
from sgl_rocm_kv import hip

pytestmark = pytest.mark.gpu
BF16_U = 2.0 ** -8   # unit roundoff of bf16 (8-bit significand, round to nearest)
FP32_TERMS = 2.0 ** -12   # the fp32 accumulation terms, times sum_i w_i |v_i|
FP16_RECORDS = 2.0 ** -11   # the latent body's scaled fp16 split records


def _latent(dk, dv):
    """Shapes the latent body takes: it keeps split records in scaled fp16
    and, when the plan asks for fast weights, rounds each weight to one
    bf16."""
    return 512 < dk <= 576 and dv == 512


def _bound(want, absw, latent, fast=False):
    """The error model's bound on |got - want| per output element."""
    weights = FP32_TERMS
    if latent:
        weights += FP16_RECORDS + (BF16_U if fast else 0.0)
    return BF16_U * np.abs(want) + weights * absw + 1e-6


def _check(got, want, case, label=""):
    """Every element within the error model's bound; prints the largest
    error and its largest ratio to the bound."""
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0].split("::")[-1]
    label = f"{test} {label}".strip()
    absw = case.absw
    bound = _bound(want, absw, _latent(case.dk, case.dv), case.fast)
    err = np.abs(np.asarray(got, np.float64) - want)
    ratio = err / bound
    worst = np.unravel_index(int(np.argmax(ratio)), ratio.shape)
    _say(f"accuracy {label}: max |d| {err.max():.3g}, max |d|/bound {ratio.max():.3f}, "
         f"max |d|/|want| (|want| > 0.1) {(err / np.maximum(np.abs(want), 0.1)).max():.3g}, "
         f"bound median {np.median(bound):.3g} max {bound.max():.3g}")
    assert (err <= bound).all(), (f"{label}: |d| {err[worst]:.3g} > bound {bound[worst]:.3g} at {worst} "
                                  f"(got {got[worst]}, want {want[worst]}, sum w|v| {absw[worst]:.3g})")


def _say(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def k():
    if hip.device_count() == 0:
        pytest.fail("no GPU visible: the gpu tests need an MI355X")
    ctx = kv.RocmKvPairCopyKernels(0)
    yield ctx
    ctx.close()


def _bf16_normal(rng, n):
    return oracle.f32_to_bf16(rng.standard_normal(n).astype(np.float32))


class _Case:
    """A pool layout (uniform K/V or an MLA pair), seeded bf16 contents,
    queries and metadata; runs the kernel and the oracle."""

    def __init__(self, rng, *, P, L, H, dk, dv, qh, pages, layer, hnd=False):
        kb, vb = H * dk * 2, H * dv * 2
        rt = kv.KvCacheRuntimeLayout("bf16", P, L, H, dk, 2, L * (kb + vb), L * (kb + vb) * P)
        if kb == vb:
            self.layout = kv.PagedKvCacheLayout.new(rt, pages)
        else:
            self.layout = kv.PagedKvCacheLayout.new_with_tensor_pair(rt, pages, kb, vb)
        self.P, self.H, self.dk, self.dv, self.qh, self.layer, self.hnd = P, H, dk, dv, qh, layer, hnd
        self.fast = False
        self.pool_h = _bf16_normal(rng, self.layout.total_byte_len // 2).view(np.uint8)
        self.pool = hip.DeviceBuffer.from_array(self.pool_h)

    def run(self, k, queries, qri, qsl, rso, slots, scale, max_len=0, use_async=False, exact=False,
            fast=False):
        self.fast = fast
        qri = np.asarray(qri, np.uint32)
        qsl = np.asarray(qsl, np.uint64)
        rso = np.asarray(rso, np.uint64)
        slots = np.asarray(slots, np.uint64)
        plan = kv.PagedAttentionPlan.for_layer(self.layout, self.layer, len(qri), len(rso) - 1,
                                               len(slots), self.qh, scale,
                                               kv.HND if self.hnd else kv.NHD, exact_weights=exact,
                                               fast_weights=fast)
        out = hip.DeviceBuffer(plan.output_required_bytes)
        out.upload(np.zeros(plan.output_required_bytes, np.uint8))
        bufs = dict(queries=hip.DeviceBuffer.from_array(queries),
                    query_request_indices=hip.DeviceBuffer.from_array(qri),
                    query_sequence_lengths=hip.DeviceBuffer.from_array(qsl),
                    request_slot_offsets=hip.DeviceBuffer.from_array(rso),
                    sequence_slots=hip.DeviceBuffer.from_array(slots), pool=self.pool, output=out)
        if use_async:
            k.paged_attention_async(plan, max_sequence_length=max_len, **bufs)
            k.check_errors()
        else:
            k.paged_attention(plan, max_sequence_length=max_len, **bufs)
        got = oracle.bf16_to_f32(out.download().view(np.uint16)).reshape(len(qri), self.qh, self.dv)
        want, flags, self.absw = oracle.paged_attention(
            self.pool_h, queries, qri, qsl, rso, slots, page_size=self.P,
            page_stride=plan.page_stride_bytes, key_offset=plan.key_in_page_offset,
            value_offset=plan.value_in_page_offset, kv_heads=self.H, dk=self.dk, dv=self.dv,
            scale=scale, slot_count=self.layout.slot_count, hnd=self.hnd, with_abs=True)
        assert flags == 0
        return got, want


def _random_batch(rng, requests, max_len, slot_count, min_len=1):
    lens = rng.integers(min_len, max_len + 1, size=requests)
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.choice(slot_count, size=int(rso[-1]), replace=False).astype(np.uint64)
    return lens, rso, slots


def test_reference_scheduler_metadata(k, goldens):
    """The two-request causal prefill of the reference's attention test:
    query_request_indices [0,0,0,1,1], lengths [1,2,3,1,2], slots 0..4 on a
    P4 L2 H2 D8 pool, layer 1, 4 query heads, scale 1/sqrt(8)."""
    f = goldens["paged_attention_plan"]["from_layout"]
    rng = np.random.default_rng(1)
    c = _Case(rng, P=4, L=2, H=2, dk=8, dv=8, qh=4, pages=2, layer=1)
    m = f["metadata"]
    q = _bf16_normal(rng, 5 * 4 * 8).reshape(5, 4, 8)
    got, want = c.run(k, q, m["query_request_indices"], m["query_sequence_lengths"],
                      m["request_slot_offsets"], m["sequence_slots"], 1.0 / math.sqrt(8.0))
    _check(got, want, c)


@pytest.mark.parametrize("hnd,P", [(False, 16), (True, 64), (False, 1), (True, 16), (True, 2), (True, 48)])
def test_llama3_8b_decode(k, hnd, P):
    """32 query heads over 8 KV heads of 128 dims; 16 requests of up to
    1,500 tokens, one decode query each (length = the whole sequence)."""
    rng = np.random.default_rng(10 + P)
    pages = -(-16 * 1500 // P) + 4
    c = _Case(rng, P=P, L=2, H=8, dk=128, dv=128, qh=32, pages=pages, layer=1, hnd=hnd)
    lens, rso, slots = _random_batch(rng, 16, 1500, c.layout.slot_count)
    q = _bf16_normal(rng, 16 * 32 * 128).reshape(16, 32, 128)
    _say(f"llama3-8b decode P={P} hnd={hnd} tokens={int(rso[-1])}")
    got, want = c.run(k, q, np.arange(16), lens, rso, slots, 1.0 / math.sqrt(128), max_len=1500)
    _check(got, want, c)


@pytest.mark.parametrize("H,qh,P,hnd,nreq,max_len", [
    (8, 32, 16, False, 16, 1500),   # Llama-3.2-1B: 32 query heads over 8 KV heads
    (2, 14, 64, True, 8, 3000),     # Qwen2-0.5B: groups of 7 heads, head-major pages
    (8, 32, 1, False, 4, 300),      # one-token pages
    (1, 16, 16, False, 2, 9000),    # long sequences: many splits of the slot table's size
])
def test_dims64_decode(k, H, qh, P, hnd, nreq, max_len):
    """Decode with K and V head dims 64 (the dims-64 staged body)."""
    rng = np.random.default_rng(64 + P + qh)
    pages = -(-nreq * max_len // P) + 4
    c = _Case(rng, P=P, L=2, H=H, dk=64, dv=64, qh=qh, pages=pages, layer=1, hnd=hnd)
    lens, rso, slots = _random_batch(rng, nreq, max_len, c.layout.slot_count)
    q = _bf16_normal(rng, nreq * qh * 64).reshape(nreq, qh, 64)
    _say(f"dims-64 decode H={H} qh={qh} P={P} hnd={hnd} tokens={int(rso[-1])}")
    got, want = c.run(k, q, np.arange(nreq), lens, rso, slots, 1.0 / math.sqrt(64), max_len=max_len)
    _check(got, want, c)


@pytest.mark.parametrize("H,qh,P,hnd,nreq,max_len", [
    (2, 8, 64, False, 16, 1500),   # Qwen3.5's full-attention layers: 8 query heads over 2 KV heads
    (2, 8, 16, True, 6, 4000),     # head-major pages, long sequences split several times
    (2, 8, 64, False, 1, 3000),    # one query: 64-token chunks, many splits
    (4, 64, 64, True, 3, 700),     # groups of 16 query heads
])
def test_dims256_decode(k, H, qh, P, hnd, nreq, max_len):
    """Decode with K and V head dims 256 (the dims-256 staged body): the
    reference's Qwen3.5 configuration (model_registry.rs:628-660) has
    head_dim 256, 8 query heads and 2 KV heads."""
    rng = np.random.default_rng(256 + P + qh + nreq)
    pages = -(-nreq * max_len // P) + 4
    c = _Case(rng, P=P, L=2, H=H, dk=256, dv=256, qh=qh, pages=pages, layer=1, hnd=hnd)
    lens, rso, slots = _random_batch(rng, nreq, max_len, c.layout.slot_count)
    q = _bf16_normal(rng, nreq * qh * 256).reshape(nreq, qh, 256)
    _say(f"dims-256 decode H={H} qh={qh} P={P} hnd={hnd} tokens={int(rso[-1])}")
    got, want = c.run(k, q, np.arange(nreq), lens, rso, slots, 1.0 / math.sqrt(256), max_len=max_len)
    _check(got, want, c)


def test_long_sequence_is_split_and_combined(k):
    """One request of 20,000 tokens (many splits through the combine kernel)
    and a short one in the same launch; the short query's sequence ends
    inside the first split."""
    rng = np.random.default_rng(2)
    c = _Case(rng, P=16, L=1, H=8, dk=128, dv=128, qh=32, pages=1300, layer=0)
    lens = np.array([20000, 40])
    rso = np.array([0, 20000, 20040], np.uint64)
    slots = rng.choice(c.layout.slot_count, size=20040, replace=False).astype(np.uint64)
    q = _bf16_normal(rng, 3 * 32 * 128).reshape(3, 32, 128)
    _say("split attention: 20,000 + 40 tokens")
    got, want = c.run(k, q, [0, 1, 0], [20000, 40, 77], rso, slots, 1.0 / math.sqrt(128),
                      max_len=20000)
    _check(got, want, c)
    # The same launch without the length hint (the split comes from the
    # total slot count) gives the same result.
    got2, _ = c.run(k, q, [0, 1, 0], [20000, 40, 77], rso, slots, 1.0 / math.sqrt(128))
    _check(got2, want, c, 'no length hint')


@pytest.mark.parametrize("dk,dv,qh,H", [(128, 128, 32, 8), (64, 64, 16, 2), (256, 256, 8, 2),
                                        (576, 512, 128, 1)])
def test_split_records_are_each_counted_once(k, dk, dv, qh, H):
    """Values that are constant over 256-token blocks (+-4 plus a little
    noise, a random sign per block) make each split's share of the output
    O(1): a split record that the combine dropped or merged twice would move
    the output by about 4 x that split's weight, far past the error bound.
    24 queries over one 20,000-token request take every count of splits
    from 1 to all of them (so every remainder of the combine's groups of
    eight), on the staged bodies (dims 128, 64, 256) and the latent MLA body."""
    rng = np.random.default_rng(dk + 31)
    n = 20000
    c = _Case(rng, P=64, L=1, H=H, dk=dk, dv=dv, qh=qh, pages=-(-n // 64) + 4, layer=0)
    slots = rng.choice(c.layout.slot_count, size=n, replace=False).astype(np.uint64)
    # Block-constant values: token j of the request (slot slots[j]) gets
    # sign_b * 4 + N(0, 1)/16 in every value dim, b = j // 256.
    pool16 = c.pool_h.view(np.uint16)
    plan = kv.PagedAttentionPlan.for_layer(c.layout, 0, 1, 1, n, qh, 0.1)
    sign = rng.choice([-4.0, 4.0], size=-(-n // 256))
    vals = sign[np.arange(n) // 256][:, None] + rng.standard_normal((n, H * dv)) / 16
    vbits = oracle.f32_to_bf16(vals.astype(np.float32))
    page, pos = slots.astype(np.int64) // 64, slots.astype(np.int64) % 64
    vstart = (page * plan.page_stride_bytes + plan.value_in_page_offset + pos * H * dv * 2) // 2
    pool16[vstart[:, None] + np.arange(H * dv)[None, :]] = vbits
    c.pool.upload(c.pool_h)
    nq = 24
    qsl = np.linspace(1, n, nq).astype(np.int64)
    q = _bf16_normal(rng, nq * qh * dk).reshape(nq, qh, dk)
    _say(f"split records counted once: dk={dk} dv={dv} qh={qh}, {nq} queries up to {n} tokens")
    got, want = c.run(k, q, np.zeros(nq, int), qsl, [0, n], slots, 1.0 / math.sqrt(dk), max_len=n)
    _check(got, want, c)


@pytest.mark.parametrize("H,qh,dk,dv,hnd", [
    (2, 64, 128, 128, False),    # group of 32: two head groups per KV head
    (1, 16, 576, 512, False),    # MLA widths (DeepSeek pair): dv spans 4 blocks
    (1, 20, 576, 512, True),     # MLA widths, head-major, group not a multiple of 16
    (1, 32, 256, 256, False),    # dims 256, two head groups: the wide body
    (2, 6, 12, 4, False),        # odd widths: element-wise loads
    (3, 9, 40, 24, True),        # dims not multiples of 32
])
def test_shapes(k, H, qh, dk, dv, hnd):
    rng = np.random.default_rng(dk + dv + qh)
    P = 16
    c = _Case(rng, P=P, L=2, H=H, dk=dk, dv=dv, qh=qh, pages=200, layer=1, hnd=hnd)
    lens, rso, slots = _random_batch(rng, 5, 600, c.layout.slot_count)
    nq = 7
    qri = rng.integers(0, 5, size=nq)
    qsl = np.array([rng.integers(1, lens[r] + 1) for r in qri])
    q = _bf16_normal(rng, nq * qh * dk).reshape(nq, qh, dk)
    _say(f"attention shape H={H} qh={qh} dk={dk} dv={dv} hnd={hnd}")
    got, want = c.run(k, q, qri, qsl, rso, slots, 1.0 / math.sqrt(dk), max_len=600)
    _check(got, want, c)


@pytest.mark.parametrize("dk,dv,P,hnd", [(128, 128, 64, False), (128, 128, 64, True), (64, 64, 16, False),
                                         (256, 256, 64, False), (576, 512, 16, False)])
def test_slots_outside_the_sequences_hold_nan(k, dk, dv, P, hnd):
    """Every pool byte the queries do not attend is a NaN pattern: padded
    tokens of the last block (lengths not a multiple of 32) and split ends
    must contribute exact zeros, never garbage, on the staged bodies (dims
    128 with K in LDS and, head-major, in registers; 64; 256) and the latent
    one (MLA widths). With one KV head, head-major and token-major pages
    hold the same bytes."""
    rng = np.random.default_rng(dk + P + hnd)
    c = _Case(rng, P=P, L=1, H=1, dk=dk, dv=dv, qh=8, pages=120, layer=0, hnd=hnd)
    lens = np.array([1, 31, 33, 700, 1001])
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.choice(c.layout.slot_count, size=int(rso[-1]), replace=False).astype(np.uint64)
    pool16 = c.pool_h.view(np.uint16)
    keep = np.zeros(c.layout.slot_count, bool)
    keep[slots.astype(np.int64)] = True
    plan = kv.PagedAttentionPlan.for_layer(c.layout, 0, 5, 5, len(slots), 8, 0.1)
    per_slot = np.arange(c.layout.total_byte_len // 2)
    page_elems = plan.page_stride_bytes // 2
    tok = (per_slot % page_elems)
    key_e, val_e = plan.key_in_page_offset // 2, plan.value_in_page_offset // 2
    in_key = (tok >= key_e) & (tok < key_e + P * dk)
    in_val = (tok >= val_e) & (tok < val_e + P * dv)
    slot_of = np.where(in_key, (per_slot // page_elems) * P + (tok - key_e) // dk,
                       (per_slot // page_elems) * P + (tok - val_e) // max(dv, 1))
    nan_mask = ~((in_key | in_val) & keep[np.clip(slot_of, 0, c.layout.slot_count - 1)])
    pool16[nan_mask] = 0x7FC1
    c.pool.upload(c.pool_h)
    q = _bf16_normal(rng, 5 * 8 * dk).reshape(5, 8, dk)
    _say(f"nan-filled pool dk={dk} dv={dv} P={P} hnd={hnd}")
    got, want = c.run(k, q, np.arange(5), lens, rso, slots, 1.0 / math.sqrt(dk), max_len=1001)
    assert np.isfinite(want).all() and np.isfinite(got).all()
    _check(got, want, c)


@pytest.mark.parametrize("qh,hnd", [(128, False), (64, True), (48, False), (16, False), (8, True)])
def test_mla_many_heads(k, qh, hnd):
    """DeepSeek-V3's MLA decode as the reference calls it (cuda_mla.rs:273-294):
    every query head over one latent KV head, K 576 and V 512 wide (the
    reference's pair layout), sequences long enough to split, partial head
    blocks (48 heads) and head-major pages."""
    rng = np.random.default_rng(qh + 5)
    c = _Case(rng, P=64, L=2, H=1, dk=576, dv=512, qh=qh, pages=200, layer=1, hnd=hnd)
    lens, rso, slots = _random_batch(rng, 6, 2000, c.layout.slot_count)
    q = _bf16_normal(rng, 6 * qh * 576).reshape(6, qh, 576)
    _say(f"mla decode qh={qh} hnd={hnd} tokens={int(rso[-1])}")
    got, want = c.run(k, q, np.arange(6), lens, rso, slots, 1.0 / math.sqrt(576), max_len=2000,
                      use_async=hnd)
    _check(got, want, c)


@pytest.mark.parametrize("D,nq,hnd", [(128, 1, False), (128, 2, False), (64, 1, False), (64, 3, False),
                                      (128, 1, True), (128, 3, True)])
def test_staged_small_batches(k, D, nq, hnd):
    """One to three GQA decode queries (32 heads over 8 KV heads): the
    staged bodies split each 3,000-token sequence into 64-token chunks (up
    to 47 splits; 128-token chunks for the body with K in registers, which
    head-major pages at dims 128 take), which the combine merges several
    groups of eight at a time in parallel thread sets."""
    rng = np.random.default_rng(D + nq + hnd)
    c = _Case(rng, P=16, L=2, H=8, dk=D, dv=D, qh=32, pages=600, layer=1, hnd=hnd)
    lens = np.array([3000, 1777, 2500][:nq])
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.choice(c.layout.slot_count, size=int(rso[-1]), replace=False).astype(np.uint64)
    q = _bf16_normal(rng, nq * 32 * D).reshape(nq, 32, D)
    _say(f"staged small batch: dims {D}, {nq} queries, hnd={hnd}, lengths {list(lens)}")
    got, want = c.run(k, q, np.arange(nq), lens, rso, slots, 1.0 / math.sqrt(D), max_len=int(lens.max()))
    _check(got, want, c)


@pytest.mark.parametrize("nq", [1, 2, 3])
def test_latent_small_batches(k, nq):
    """One to three MLA decode queries: the latent body's chunks shrink to
    64 (one query) or 128 tokens, so a 3,000-token sequence takes up to 47
    splits, which the combine merges four groups of eight at a time."""
    rng = np.random.default_rng(nq + 90)
    c = _Case(rng, P=64, L=2, H=1, dk=576, dv=512, qh=128, pages=160, layer=1)
    lens = np.array([3000, 1777, 2500][:nq])
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.choice(c.layout.slot_count, size=int(rso[-1]), replace=False).astype(np.uint64)
    q = _bf16_normal(rng, nq * 128 * 576).reshape(nq, 128, 576)
    _say(f"latent small batch: {nq} queries, lengths {list(lens)}")
    got, want = c.run(k, q, np.arange(nq), lens, rso, slots, 1.0 / math.sqrt(576), max_len=int(lens.max()))
    _check(got, want, c)


@pytest.mark.parametrize("nq,qh,hnd,max_len", [
    (6, 128, False, 2000),   # DeepSeek's 128 heads, split sequences
    (4, 48, True, 2000),     # partial head blocks, head-major pages
    (1, 128, False, 3000),   # one query: 64-token chunks, 47 splits
    (9, 72, True, 250),      # one split: no records, no combine
])
def test_latent_weights(k, nq, qh, hnd, max_len):
    """The latent body's default plan feeds each weight as hi + lo bf16
    values, so the output meets the bound without the 2^-8 sum w|v| term;
    a plan that names ATTN_EXACT_WEIGHTS gives the same bits; a plan with
    ATTN_FAST_WEIGHTS (one bf16 per weight) meets the looser bound."""
    rng = np.random.default_rng(qh + nq + 300)
    c = _Case(rng, P=64, L=2, H=1, dk=576, dv=512, qh=qh, pages=-(-nq * max_len // 64) + 8,
              layer=1, hnd=hnd)
    lens, rso, slots = _random_batch(rng, nq, max_len, c.layout.slot_count)
    if nq == 1:
        lens[:] = max_len
        rso = np.array([0, max_len], np.uint64)
        slots = rng.choice(c.layout.slot_count, size=max_len, replace=False).astype(np.uint64)
    q = _bf16_normal(rng, nq * qh * 576).reshape(nq, qh, 576)
    _say(f"latent weights: {nq} queries, qh={qh} hnd={hnd} tokens={int(rso[-1])}")
    args = (k, q, np.arange(nq), lens, rso, slots, 1.0 / math.sqrt(576))
    got, want = c.run(*args, max_len=int(lens.max()))
    _check(got, want, c, "default")
    got_x, _ = c.run(*args, max_len=int(lens.max()), exact=True)
    np.testing.assert_array_equal(got_x, got)
    got_f, _ = c.run(*args, max_len=int(lens.max()), fast=True)
    _check(got_f, want, c, "fast")


def test_latent_weights_cancellation(k):
    """Values of +-4 (a random sign per token) over 4..64 tokens: the
    output is a small difference of large terms, where rounding each weight
    to one bf16 (about 2^-9 relative) moves the bf16 output by an ulp for
    roughly one element in five, and hi + lo weights for almost none. Each
    sequence fits one split, so no fp16 record rounds in between. The
    default plan must round to the oracle's bf16 value in at least 99 % of
    the elements and, by that count, be several times closer than a plan
    with ATTN_FAST_WEIGHTS (which shows that the flag reaches the kernel)."""
    rng = np.random.default_rng(4242)
    nq, qh = 32, 128
    c = _Case(rng, P=64, L=1, H=1, dk=576, dv=512, qh=qh, pages=48, layer=0)
    lens = rng.integers(4, 65, size=nq)
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.choice(c.layout.slot_count, size=int(rso[-1]), replace=False).astype(np.uint64)
    pool16 = c.pool_h.view(np.uint16)
    plan = kv.PagedAttentionPlan.for_layer(c.layout, 0, nq, nq, len(slots), qh, 0.1)
    n = len(slots)
    vals = rng.choice([-4.0, 4.0], size=(n, 1)) + rng.standard_normal((n, 512)) / 16
    page, pos = slots.astype(np.int64) // 64, slots.astype(np.int64) % 64
    vstart = (page * plan.page_stride_bytes + plan.value_in_page_offset + pos * 512 * 2) // 2
    pool16[vstart[:, None] + np.arange(512)[None, :]] = oracle.f32_to_bf16(vals.astype(np.float32))
    c.pool.upload(c.pool_h)
    # Scores of a few log2 units, so no single token's weight dominates.
    q = oracle.f32_to_bf16(2.0 * rng.standard_normal(nq * qh * 576).astype(np.float32)).reshape(nq, qh, 576)
    args = (k, q, np.arange(nq), lens, rso, slots, 1.0 / math.sqrt(576))
    got_e, want = c.run(*args, max_len=64)
    _check(got_e, want, c, "default")
    got_f, _ = c.run(*args, max_len=64, fast=True)
    _check(got_f, want, c, "fast")
    rounded = oracle.bf16_to_f32(oracle.f32_to_bf16(want.astype(np.float32)))
    off_e = float(np.mean(got_e != rounded))
    off_f = float(np.mean(got_f != rounded))
    _say(f"cancellation: elements off the oracle's bf16 value: default {off_e:.4f}, fast {off_f:.4f}")
    assert off_e <= 0.01
    assert off_e * 4 < off_f


@pytest.mark.parametrize("H,qh,dk,hnd", [
    (2, 256, 576, False),   # two KV heads, a full 128-head block each
    (1, 160, 576, True),    # two head blocks, the second holding 32 heads
    (1, 100, 544, False),   # the last wave with 4 heads; K rows with 32 of 64 tail dims
])
def test_latent_shapes(k, H, qh, dk, hnd):
    """The latent body (V rows of 512, K rows of 520..576 dims) beyond
    DeepSeek's exact shape: several KV heads, more than 128 query heads per
    KV head, waves with fewer than 32 heads, and K rows whose last 64 dims
    are only partly there (the rest must read as zeros)."""
    rng = np.random.default_rng(qh + dk)
    c = _Case(rng, P=64, L=2, H=H, dk=dk, dv=512, qh=qh, pages=80, layer=1, hnd=hnd)
    lens, rso, slots = _random_batch(rng, 3, 1200, c.layout.slot_count)
    q = _bf16_normal(rng, 3 * qh * dk).reshape(3, qh, dk)
    _say(f"latent shape H={H} qh={qh} dk={dk} hnd={hnd} tokens={int(rso[-1])}")
    got, want = c.run(k, q, np.arange(3), lens, rso, slots, 1.0 / math.sqrt(dk), max_len=1200)
    _check(got, want, c)


@pytest.mark.parametrize("qh,hnd", [(128, False), (72, True)])
def test_latent_one_split(k, qh, hnd):
    """MLA decode with sequences of at most 256 tokens: one split, so the
    latent body writes the bf16 output itself (no split records, no
    combine pass), with blocks past each sequence's end masked."""
    rng = np.random.default_rng(qh + 7)
    c = _Case(rng, P=64, L=2, H=1, dk=576, dv=512, qh=qh, pages=40, layer=0, hnd=hnd)
    lens, rso, slots = _random_batch(rng, 9, 250, c.layout.slot_count)
    q = _bf16_normal(rng, 9 * qh * 576).reshape(9, qh, 576)
    _say(f"latent one split qh={qh} hnd={hnd} lens={lens.tolist()}")
    got, want = c.run(k, q, np.arange(9), lens, rso, slots, 1.0 / math.sqrt(576), max_len=250)
    _check(got, want, c)


@pytest.mark.parametrize("dk,dv,qh,hnd", [(576, 512, 32, False), (128, 128, 48, True)])
def test_wide_reference_outrun(k, dk, dv, qh, hnd):
    """Queries 100 times larger spread the scores over hundreds of log2
    units, so later blocks of a split exceed its first block's maximum by
    far more than the wide bodies' fixed reference allows: the workgroup
    must notice and recompute the split with per-block rescaling (a clamped
    fast path would give visibly wrong weights)."""
    rng = np.random.default_rng(dk + qh)
    c = _Case(rng, P=64, L=2, H=1, dk=dk, dv=dv, qh=qh, pages=120, layer=0, hnd=hnd)
    lens, rso, slots = _random_batch(rng, 5, 1500, c.layout.slot_count, min_len=600)
    q = oracle.f32_to_bf16(100.0 * rng.standard_normal(5 * qh * dk).astype(np.float32)).reshape(5, qh, dk)
    _say(f"wide reference outrun dk={dk} dv={dv} qh={qh} hnd={hnd}")
    got, want = c.run(k, q, np.arange(5), lens, rso, slots, 1.0 / math.sqrt(dk), max_len=1500)
    assert np.isfinite(got).all()
    _check(got, want, c)


@pytest.mark.parametrize("H,dk,dv", [(1, 576, 512), (8, 128, 128)])
def test_wide_unaligned_queries(k, H, dk, dv):
    """A query buffer that is only 2-byte aligned: the latent, wide and
    staged bodies hold queries as 16-byte vectors, so the launch must take
    the generic body (MLA widths) or the pipelined one (dims 128), with the
    same results."""
    rng = np.random.default_rng(41 + dk)
    c = _Case(rng, P=64, L=2, H=H, dk=dk, dv=dv, qh=32, pages=60 * H, layer=1)
    lens, rso, slots = _random_batch(rng, 3, 900, c.layout.slot_count)
    q = _bf16_normal(rng, 3 * 32 * dk).reshape(3, 32, dk)
    plan = kv.PagedAttentionPlan.for_layer(c.layout, 1, 3, 3, len(slots), 32, 1.0 / math.sqrt(dk))
    qbuf = hip.DeviceBuffer(q.nbytes + 2)
    qbuf.upload(np.concatenate([np.zeros(1, np.uint16), q.reshape(-1)]).view(np.uint8))
    out = hip.DeviceBuffer(plan.output_required_bytes)
    _say(f"queries at a 2-byte offset, H={H} dk={dk} dv={dv}")
    k.paged_attention(plan, max_sequence_length=900, queries=qbuf, queries_offset=2,
                      query_request_indices=hip.DeviceBuffer.from_array(np.arange(3, dtype=np.uint32)),
                      query_sequence_lengths=hip.DeviceBuffer.from_array(lens.astype(np.uint64)),
                      request_slot_offsets=hip.DeviceBuffer.from_array(rso),
                      sequence_slots=hip.DeviceBuffer.from_array(slots), pool=c.pool, output=out)
    got = oracle.bf16_to_f32(out.download().view(np.uint16)).reshape(3, 32, dv)
    want, flags, absw = oracle.paged_attention(
        c.pool_h, q, np.arange(3), lens, rso, slots, page_size=64, page_stride=plan.page_stride_bytes,
        key_offset=plan.key_in_page_offset, value_offset=plan.value_in_page_offset, kv_heads=H, dk=dk,
        dv=dv, scale=1.0 / math.sqrt(dk), slot_count=c.layout.slot_count, with_abs=True)
    assert flags == 0
    c.absw = absw
    _check(got, want, c)


@pytest.mark.parametrize("dk,dv,qh,max_len", [
    (576, 512, 16, 4300),    # latent body, 4,096-token table
    (128, 128, 32, 20000),   # wide body, 4,096-token table
    (128, 128, 16, 9000),    # staged body, 1,024-token table
    (64, 64, 16, 9000),      # dims-64 staged body, 1,024-token table
])
def test_wide_chunk_capped_by_slot_table(k, dk, dv, qh, max_len):
    """Enough queries to fill the GPU with few splits (256 workgroups) and
    sequences longer than the body's slot table allows per split: the host
    must cap the chunk, so a query takes several splits, and the
    shorter ones use fewer of them than the launch has. Sequences reuse the
    rows of a small pool (slots drawn with replacement, as a slot list may
    repeat them). A sample of the queries is checked."""
    rng = np.random.default_rng(43 + dk)
    nq = 256
    c = _Case(rng, P=64, L=1, H=1, dk=dk, dv=dv, qh=qh, pages=48, layer=0)
    lens = rng.integers(max_len - 300, max_len + 1, size=nq)
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.integers(0, c.layout.slot_count, size=int(rso[-1])).astype(np.uint64)
    q = _bf16_normal(rng, nq * qh * dk).reshape(nq, qh, dk)
    plan = kv.PagedAttentionPlan.for_layer(c.layout, 0, nq, nq, len(slots), qh, 1.0 / math.sqrt(dk))
    out = hip.DeviceBuffer(plan.output_required_bytes)
    _say(f"chunk capped by the slot table: {nq} queries x up to {lens.max()} tokens, dk {dk} qh {qh}")
    k.paged_attention(plan, max_sequence_length=int(lens.max()), queries=hip.DeviceBuffer.from_array(q),
                      query_request_indices=hip.DeviceBuffer.from_array(np.arange(nq, dtype=np.uint32)),
                      query_sequence_lengths=hip.DeviceBuffer.from_array(lens.astype(np.uint64)),
                      request_slot_offsets=hip.DeviceBuffer.from_array(rso),
                      sequence_slots=hip.DeviceBuffer.from_array(slots), pool=c.pool, output=out)
    got = oracle.bf16_to_f32(out.download().view(np.uint16)).reshape(nq, qh, dv)
    pick = np.array([0, int(np.argmax(lens)), int(np.argmin(lens)), 101, nq - 1])
    want, flags, absw = oracle.paged_attention(
        c.pool_h, q[pick], pick, lens[pick], rso, slots, page_size=64, page_stride=plan.page_stride_bytes,
        key_offset=plan.key_in_page_offset, value_offset=plan.value_in_page_offset, kv_heads=1, dk=dk,
        dv=dv, scale=1.0 / math.sqrt(dk), slot_count=c.layout.slot_count, with_abs=True)
    assert flags == 0
    c.absw = absw
    _check(got[pick], want, c)


def _random_shape(rng):
    """One random attention problem: head dims, GQA group, page size (powers
    of two take the pipelined body, others the generic one), head layout,
    request lengths (tails not a multiple of 32), queries per request."""
    H = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 5, 8, 16, 24]))
    dk = int(rng.choice([8, 16, 40, 64, 96, 128, 192]))
    dv = dk if rng.random() < 0.7 else int(rng.choice([8, 64, 128, 136]))
    P = int(rng.choice([1, 3, 8, 16, 64]))
    hnd = bool(rng.random() < 0.5)
    requests = int(rng.integers(1, 6))
    lens = rng.integers(1, 700, size=requests)
    return dict(H=H, qh=H * group, dk=dk, dv=dv, P=P, hnd=hnd, lens=lens)


@pytest.mark.parametrize("seed", range(12))
def test_random_shapes(k, seed):
    rng = np.random.default_rng(1000 + seed)
    sh = _random_shape(rng)
    lens = sh["lens"]
    total = int(lens.sum())
    pages = -(-total // sh["P"]) + 8
    c = _Case(rng, P=sh["P"], L=2, H=sh["H"], dk=sh["dk"], dv=sh["dv"], qh=sh["qh"], pages=pages, layer=1,
              hnd=sh["hnd"])
    rso = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    slots = rng.choice(c.layout.slot_count, size=total, replace=False).astype(np.uint64)
    nq = int(rng.integers(1, 9))
    qri = rng.integers(0, len(lens), size=nq)
    qsl = np.array([rng.integers(1, lens[r] + 1) for r in qri])
    q = _bf16_normal(rng, nq * sh["qh"] * sh["dk"]).reshape(nq, sh["qh"], sh["dk"])
    _say(f"random attention seed={seed} {dict((k_, v) for k_, v in sh.items() if k_ != 'lens')} "
         f"lens={list(lens)} queries={nq}")
    got, want = c.run(k, q, qri, qsl, rso, slots, 1.0 / math.sqrt(sh["dk"]), max_len=int(lens.max()),
                      use_async=bool(seed % 2))
    _check(got, want, c)


def test_metadata_errors(k):
    """Bad request index, empty or overlong length, and a slot past the pool
    raise DeviceMetadataInvalid with the reference's flag values."""
    rng = np.random.default_rng(4)
    c = _Case(rng, P=16, L=1, H=2, dk=64, dv=64, qh=4, pages=4, layer=0)
    q = _bf16_normal(rng, 2 * 4 * 64).reshape(2, 4, 64)
    cases = [([0, 1], [3, 3], [0, 3], [0, 1, 2], 0x1),
             ([0, 0], [3, 0], [0, 3], [0, 1, 2], 0x2),
             ([0, 0], [3, 4], [0, 3], [0, 1, 2], 0x2),
             ([0, 0], [3, 2], [0, 3], [0, 64, 2], 0x4)]
    for qri, qsl, rso, slots, want in cases:
        plan = kv.PagedAttentionPlan.for_layer(c.layout, 0, 2, len(rso) - 1, len(slots), 4, 0.125)
        out = hip.DeviceBuffer(plan.output_required_bytes)
        with pytest.raises(kv.KvError) as ei:
            k.paged_attention(plan, queries=hip.DeviceBuffer.from_array(q),
                              query_request_indices=hip.DeviceBuffer.from_array(np.array(qri, np.uint32)),
                              query_sequence_lengths=hip.DeviceBuffer.from_array(np.array(qsl, np.uint64)),
                              request_slot_offsets=hip.DeviceBuffer.from_array(np.array(rso, np.uint64)),
                              sequence_slots=hip.DeviceBuffer.from_array(np.array(slots, np.uint64)),
                              pool=c.pool, output=out)
        assert ei.value.variant == "DeviceMetadataInvalid" and ei.value.fields[0] == want


def test_length_above_the_stated_maximum_is_rejected(k):
    """A query longer than max_sequence_length (here 600 tokens against a
    stated 300, which the launch covers with 2 splits of 256) is reported as
    a sequence error, not truncated or combined from missing splits."""
    rng = np.random.default_rng(7)
    c = _Case(rng, P=16, L=1, H=2, dk=64, dv=64, qh=4, pages=64, layer=0)
    slots = rng.choice(c.layout.slot_count, size=600, replace=False).astype(np.uint64)
    q = _bf16_normal(rng, 2 * 4 * 64).reshape(2, 4, 64)
    plan = kv.PagedAttentionPlan.for_layer(c.layout, 0, 2, 1, 600, 4, 0.125)
    with pytest.raises(kv.KvError) as ei:
        k.paged_attention(plan, max_sequence_length=300, queries=hip.DeviceBuffer.from_array(q),
                          query_request_indices=hip.DeviceBuffer.from_array(np.zeros(2, np.uint32)),
                          query_sequence_lengths=hip.DeviceBuffer.from_array(np.array([100, 600], np.uint64)),
                          request_slot_offsets=hip.DeviceBuffer.from_array(np.array([0, 600], np.uint64)),
                          sequence_slots=hip.DeviceBuffer.from_array(slots), pool=c.pool,
                          output=hip.DeviceBuffer(plan.output_required_bytes))
    assert ei.value.variant == "DeviceMetadataInvalid" and ei.value.fields[0] == 0x2


@pytest.mark.parametrize("max_len", [0, 1500])
def test_async_launch_matches_and_reports_at_check_errors(k, max_len):
    """paged_attention_async gives the synchronous call's results (split and
    unsplit launches) and its metadata errors surface at check_errors."""
    rng = np.random.default_rng(8)
    c = _Case(rng, P=64, L=1, H=8, dk=128, dv=128, qh=32, pages=400, layer=0, hnd=True)
    lens, rso, slots = _random_batch(rng, 12, 1500, c.layout.slot_count)
    q = _bf16_normal(rng, 12 * 32 * 128).reshape(12, 32, 128)
    got, want = c.run(k, q, np.arange(12), lens, rso, slots, 1.0 / math.sqrt(128), max_len=max_len,
                      use_async=True)
    _check(got, want, c)
    plan = kv.PagedAttentionPlan.for_layer(c.layout, 0, 2, 1, 4, 32, 0.1, kv.HND)
    bad = dict(queries=hip.DeviceBuffer.from_array(q[:2]),
               query_request_indices=hip.DeviceBuffer.from_array(np.array([0, 3], np.uint32)),
               query_sequence_lengths=hip.DeviceBuffer.from_array(np.array([2, 2], np.uint64)),
               request_slot_offsets=hip.DeviceBuffer.from_array(np.array([0, 4], np.uint64)),
               sequence_slots=hip.DeviceBuffer.from_array(slots[:4]), pool=c.pool,
               output=hip.DeviceBuffer(plan.output_required_bytes))
    k.paged_attention_async(plan, max_sequence_length=max_len, **bad)
    with pytest.raises(kv.KvError) as ei:
        k.check_errors()
    assert ei.value.variant == "DeviceMetadataInvalid" and ei.value.fields[0] == 0x1
    k.check_errors()   # the word was cleared


def test_host_range_checks(k):
    rng = np.random.default_rng(5)
    c = _Case(rng, P=16, L=1, H=2, dk=64, dv=64, qh=4, pages=4, layer=0)
    plan = kv.PagedAttentionPlan.for_layer(c.layout, 0, 1, 1, 3, 4, 0.125)
    q = hip.DeviceBuffer(plan.query_required_bytes - 2)
    ok = dict(query_request_indices=hip.DeviceBuffer(4), query_sequence_lengths=hip.DeviceBuffer(8),
              request_slot_offsets=hip.DeviceBuffer(16), sequence_slots=hip.DeviceBuffer(24),
              pool=c.pool, output=hip.DeviceBuffer(plan.output_required_bytes))
    with pytest.raises(kv.KvError) as ei:
        k.paged_attention(plan, queries=q, **ok)
    assert ei.value.code == 11 and ei.value.name == "queries"
    # A plan edited after plan_new to carry an unknown flag is refused at
    # enqueue, before any buffer is read.
    known = kv.ATTN_EXACT_WEIGHTS | kv.ATTN_FAST_WEIGHTS
    for bad in (4, known):   # an unknown bit; exact and fast at once
        plan._c.config.flags = bad
        with pytest.raises(kv.KvError) as ei:
            k.paged_attention(plan, queries=hip.DeviceBuffer(plan.query_required_bytes), **ok)
        assert ei.value.name == "flags" and ei.value.fields[:2] == (bad, known)


def test_reads_an_hnd_pool_written_by_the_transfer_kernels(k):
    """Prefill pool (P=1 NHD) -> decode pool (P=64 HND) with transfer_layers,
    then attention over the decode pool's HND pages equals attention over
    the prefill pool's NHD pages for the same tokens."""
    rng = np.random.default_rng(6)
    L, H, D, qh, n = 2, 8, 128, 32, 3000
    src = _Case(rng, P=1, L=L, H=H, dk=D, dv=D, qh=qh, pages=4096, layer=1)
    dst = _Case(rng, P=64, L=L, H=H, dk=D, dv=D, qh=qh, pages=64, layer=1, hnd=True)
    src_slots = rng.choice(src.layout.slot_count, size=n, replace=False).astype(np.uint64)
    table = rng.permutation(dst.layout.page_count)[: -(-n // 64)]
    dst_slots = (table[np.arange(n) // 64] * 64 + np.arange(n) % 64).astype(np.uint64)
    ss, ds = hip.DeviceBuffer.from_array(src_slots), hip.DeviceBuffer.from_array(dst_slots)
    sv = src.layout.pool_view(src.pool.ptr, src.pool.nbytes, 0, kv.NHD, H)
    dv = dst.layout.pool_view(dst.pool.ptr, dst.pool.nbytes, 0, kv.HND, H)
    k.transfer_layers(sv, src.layout.bytes_per_layer_page, L, kv.device_buffer(ss.ptr, ss.nbytes), n,
                      dv, dst.layout.bytes_per_layer_page, kv.device_buffer(ds.ptr, ds.nbytes))
    k.check_errors()
    dst.pool_h = dst.pool.download()
    q = _bf16_normal(rng, 4 * qh * D).reshape(4, qh, D)
    qsl = [n, 1, 1777, 64]
    got_src, want = src.run(k, q, [0] * 4, qsl, [0, n], src_slots, 1.0 / math.sqrt(D), max_len=n)
    got_dst, want_dst = dst.run(k, q, [0] * 4, qsl, [0, n], dst_slots, 1.0 / math.sqrt(D), max_len=n)
    np.testing.assert_allclose(want_dst, want, rtol=1e-12, atol=1e-12)
    _check(got_dst, want, src, 'hnd pool written by the transfer (decode side)')
    _check(got_src, want, src, 'hnd pool written by the transfer (prefill side)')
