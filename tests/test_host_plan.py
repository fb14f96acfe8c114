"""The scheduler-side producers of a transfer span on the CPU: the
token-prefix cache (RadixCache, crates/sglang-srt/src/cache.rs:475-547), whose
page-aligned match becomes the span's token_offset, and the transfer plan of
a prefill batch (KvCacheTransferPlan::from_prefill_worker_batch_with_page_size,
crates/sglang-srt/src/transfer.rs:604-668).

The oracle's restatements are pinned first: against the reference's own
test values (tests/golden/reference_goldens.json), and the trie against a
brute-force dictionary of every inserted prefix. The product library is then
compared with the oracle on random batches, error variants included.
"""
import numpy as np
import pytest

import oracle
import sgl_rocm_kv as kv


def _oracle_cache(inserts):
    c = oracle.RadixCache()
    for toks, pages in inserts:
        c.insert(toks, pages)
    return c


def _product_cache(inserts):
    c = kv.RadixCache()
    for toks, pages in inserts:
        c.insert(toks, pages)
    return c


# --- the oracle against the reference's values and a brute force --------------------------

@pytest.mark.parametrize("case", ["longest_prefix", "uncached_branch", "page_aligned"])
def test_oracle_radix_cache_matches_reference_tests(goldens, case):
    g = goldens["radix_cache"][case]
    m, pages, rest = _oracle_cache(g["inserts"]).match_prefix_page_aligned(g["query"], g["page_size"])
    assert (m, pages, rest) == (g["matched"], g["pages"], g["remaining"])


def _brute_match(inserts, query, page_size):
    """Longest m such that every prefix query[:k], k <= m, was a prefix of an
    inserted sequence; its page is the one the last such insert gave it."""
    seen = {}
    for toks, pages in inserts:
        for k in range(1, len(toks) + 1):
            seen[tuple(toks[:k])] = pages[k - 1]
    m = 0
    while m < len(query) and tuple(query[: m + 1]) in seen:
        m += 1
    m = m // page_size * page_size
    return m, [seen[tuple(query[: k + 1])] for k in range(m)], list(query[m:])


def test_oracle_radix_cache_against_brute_force():
    rng = np.random.default_rng(11)
    for _ in range(200):
        inserts = []
        for _ in range(int(rng.integers(0, 6))):
            n = int(rng.integers(0, 9))
            inserts.append(([int(t) for t in rng.integers(0, 3, n)], [int(p) for p in rng.integers(0, 50, n)]))
        query = [int(t) for t in rng.integers(0, 3, int(rng.integers(0, 10)))]
        P = int(rng.integers(1, 5))
        assert _oracle_cache(inserts).match_prefix_page_aligned(query, P) == _brute_match(inserts, query, P)


def test_oracle_plan_matches_reference_delta(goldens):
    g = goldens["prefill_batch_plan"]["delta"]
    cache = _oracle_cache([g["prefix"]])
    m, _, rest = cache.match_prefix_page_aligned(g["request"], 1)
    slots = list(range(len(rest)))        # a fresh CachePageAllocator(8) hands out slots 0, 1, ...
    rc, spans = oracle.transfer_plan_from_prefill_batch([len(rest)], [m], [True], slots, 1)
    assert rc == 0 and len(spans) == 1
    _, off, count, pages, _ = spans[0]
    assert (off, count, len(pages)) == (g["token_offset"], g["token_count"], g["cache_page_count"])


def test_oracle_plan_skips_requests_without_params_but_consumes_their_pages():
    rc, spans = oracle.transfer_plan_from_prefill_batch([2, 3, 1], [0, 4, 0], [False, True, False],
                                                        [8, 9, 4, 5, 6, 7], 1)
    assert rc == 0 and [s[0] for s in spans] == [1] and spans[0][3] == [4, 5, 6]


# --- the product library ------------------------------------------------------------------

@pytest.mark.parametrize("case", ["longest_prefix", "uncached_branch", "page_aligned"])
def test_radix_cache_matches_reference_tests(goldens, case):
    g = goldens["radix_cache"][case]
    got = _product_cache(g["inserts"]).match_prefix_page_aligned(g["query"], g["page_size"])
    assert (got.matched_token_count, got.cache_pages, got.remaining_input_ids) == (
        g["matched"], g["pages"], g["remaining"])


def test_radix_cache_errors_and_clear(goldens):
    g = goldens["radix_cache"]
    c = kv.RadixCache()
    with pytest.raises(kv.KvError) as e:
        c.insert(g["length_mismatch"]["tokens"], g["length_mismatch"]["pages"])
    assert e.value.variant == g["length_mismatch"]["variant"]
    assert e.value.fields[:2] == (3, 2)
    gc = g["clear"]
    c = _product_cache(gc["inserts"])
    c.clear()
    got = c.match_prefix(gc["query"])
    assert (got.matched_token_count, got.cache_pages, got.remaining_input_ids) == (0, [], gc["remaining"])
    with pytest.raises(kv.KvError) as e:
        c.match_prefix_page_aligned([1], 0)
    assert e.value.code == kv.INVALID_ARGUMENT
    # an insert that overwrites the pages of an existing path
    c.insert([5, 6], [1, 2])
    c.insert([5, 6, 7], [3, 4, 5])
    assert c.match_prefix([5, 6, 7]).cache_pages == [3, 4, 5]
    assert c.match_prefix([]).matched_token_count == 0


def test_radix_cache_against_oracle_random():
    rng = np.random.default_rng(12)
    for _ in range(300):
        inserts = []
        for _ in range(int(rng.integers(0, 8))):
            n = int(rng.integers(0, 12))
            inserts.append(([int(t) for t in rng.integers(0, 4, n)],
                            [int(p) for p in rng.integers(0, 1 << 40, n)]))
        oc, pc = _oracle_cache(inserts), _product_cache(inserts)
        for _ in range(4):
            q = [int(t) for t in rng.integers(0, 4, int(rng.integers(0, 14)))]
            P = int(rng.integers(1, 6))
            got = pc.match_prefix_page_aligned(q, P)
            assert (got.matched_token_count, got.cache_pages, got.remaining_input_ids) == \
                oc.match_prefix_page_aligned(q, P)


def test_plan_matches_reference_delta(goldens):
    g = goldens["prefill_batch_plan"]["delta"]
    cache = _product_cache([g["prefix"]])
    m = cache.match_prefix_page_aligned(g["request"], 1)
    alloc = kv.CachePageAllocator(g["allocator_slots"])
    slots = alloc.allocate(len(m.remaining_input_ids))
    spans = kv.transfer_plan_from_prefill_batch([len(slots)], [m.matched_token_count], [1], slots, 1)
    assert len(spans) == 1
    s = spans[0]
    assert (s.token_offset, s.token_count, len(s.cache_pages)) == (
        g["token_offset"], g["token_count"], g["cache_page_count"])


def test_plan_two_requests_counts(goldens):
    g = goldens["prefill_batch_plan"]["two_requests"]
    cache = _product_cache([g["prefix"]])
    alloc = kv.CachePageAllocator(16)
    cached, inputs, slots = [], [], []
    for req in g["requests"]:
        m = cache.match_prefix_page_aligned(req, 1)
        cached.append(m.matched_token_count)
        inputs.append(len(m.remaining_input_ids))
        slots += alloc.allocate(len(m.remaining_input_ids))
    assert cached == g["cached_token_counts"] and inputs == g["input_token_counts"]
    spans = kv.transfer_plan_from_prefill_batch(inputs, cached, [1, 1], slots, 1)
    assert [(s.request_index, s.token_offset, s.token_count) for s in spans] == [(0, 2, 2), (1, 0, 2)]


def _variant(code):
    return {kv.PLAN_NON_PREFILL_BATCH: "NonPrefillBatch", kv.PLAN_ZERO_PAGE_SIZE: "ZeroPageSize",
            kv.PLAN_CACHE_PAGE_COUNT_MISMATCH: "CachePageCountMismatch",
            kv.PLAN_TRAILING_CACHE_PAGES: "TrailingCachePages",
            kv.PLAN_UNALIGNED_TOKEN_OFFSET: "UnalignedTokenOffset",
            kv.PLAN_UNALIGNED_CACHE_SLOT: "UnalignedCacheSlot",
            kv.PLAN_NON_CONTIGUOUS_CACHE_SLOTS: "NonContiguousCacheSlots"}[code]


def _product_plan(inputs, cached, pd, slots, P, prefill=True):
    try:
        spans = kv.transfer_plan_from_prefill_batch(
            inputs, cached, pd, slots, P, kv.FORWARD_PREFILL if prefill else kv.FORWARD_DECODE)
    except kv.KvError as e:
        return e.variant, None
    return 0, [(s.request_index, s.token_offset, s.token_count, s.cache_pages, s.page_indices) for s in spans]


def _oracle_plan(inputs, cached, pd, slots, P, prefill=True):
    rc, spans = oracle.transfer_plan_from_prefill_batch(inputs, cached, pd, slots, P, prefill)
    return (_variant(rc) if rc else 0), spans


def test_plan_error_variants_in_reference_order(goldens):
    cases = {
        # decode batches and a zero page size fail before any request is read
        "NonPrefillBatch": ([3], [0], [1], [0, 1, 2], 0, False),
        "ZeroPageSize": ([3], [0], [1], [0, 1, 2], 0, True),
        # a request with more tokens than pages left fails even without params
        "CachePageCountMismatch": ([2, 5], [0, 0], [1, 0], [0, 1, 2, 3], 2, True),
        "TrailingCachePages": ([2], [0], [1], [0, 1, 2, 3], 2, True),
        "UnalignedTokenOffset": ([2], [1], [1], [0, 1], 2, True),
        "UnalignedCacheSlot": ([2], [0], [1], [1, 2], 2, True),
        "NonContiguousCacheSlots": ([2], [0], [1], [0, 2], 2, True),
    }
    assert sorted(cases) == sorted(goldens["prefill_batch_plan"]["variants"])
    for variant, (inp, cached, pd, slots, P, prefill) in cases.items():
        assert _product_plan(inp, cached, pd, slots, P, prefill)[0] == variant
        assert _oracle_plan(inp, cached, pd, slots, P, prefill)[0] == variant
    # a request without params is not checked for alignment (no span is built)
    assert _product_plan([2], [1], [0], [1, 3], 2) == (0, [])


def _random_batch(rng, P):
    """A prefill batch as a scheduler builds it: prefixes of whole pages,
    uncached suffixes in fresh pages from a page allocator."""
    alloc = kv.CachePageAllocator(4096 * P, P)
    n = int(rng.integers(0, 7))
    inputs, cached, pd, slots = [], [], [], []
    for _ in range(n):
        count = int(rng.integers(0, 5 * P))
        inputs.append(count)
        cached.append(P * int(rng.integers(0, 4)))
        pd.append(int(rng.random() < 0.7))
        slots += alloc.allocate(count)
    return inputs, cached, pd, slots


def test_plan_against_oracle_random():
    rng = np.random.default_rng(13)
    for _ in range(400):
        P = int(rng.choice([1, 2, 4, 16]))
        inputs, cached, pd, slots = _random_batch(rng, P)
        # mutate a fifth of the cases into an error of one kind or another
        r = rng.random()
        if r < 0.05 and slots:
            slots = slots[:-1]
        elif r < 0.10:
            slots = slots + [7 * P]
        elif r < 0.15 and cached:
            cached[int(rng.integers(0, len(cached)))] += 1
        elif r < 0.20 and slots:
            i = int(rng.integers(0, len(slots)))
            slots[i] += 1
        want = _oracle_plan(inputs, cached, pd, slots, P)
        assert _product_plan(inputs, cached, pd, slots, P) == want, (inputs, cached, pd, slots, P)


def test_plan_spans_feed_the_span_checksum():
    """The span fields the plan yields are the checksum's inputs
    (transfer.rs:548-570): a span of the golden delta hashes to the same
    digest through either route."""
    spans = kv.transfer_plan_from_prefill_batch([2], [2], [1], [0, 1], 1)
    s = spans[0]
    a = kv.transfer_span_checksum("request", "127.0.0.1", 8998, 7, 0, s.token_offset, s.token_count, 1,
                                  s.cache_pages, s.page_indices)
    b = kv.transfer_span_checksum("request", "127.0.0.1", 8998, 7, 0, 2, 2, 1, [0, 1], [0, 1])
    assert a == b and len(a) == 64
