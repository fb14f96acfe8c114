// kv_attention.hip -- paged attention over bf16 K/V pages for gfx950, the
// reader of the pools the copy kernels write (NHD pages as the reference
// lays them out, and HND pages, which the reference cannot read).
//
// Same contract as sglang_paged_attention_bf16
// (crates/sglang-kernel/src/cuda_attention.rs:10-155): query q of request
// r attends the first query_sequence_lengths[q] slots of r's slot list with
// an fp32 online softmax, GQA head h -> KV head h / (query_heads /
// kv_heads), bf16 output rounded to nearest even. The reference runs one
// 256-thread block per (query, head), reduces each q.k dot product through
// shared memory and walks the sequence token by token. Here:
//  - a workgroup is one 64-lane wave and owns up to 16 query heads of one
//    KV head, so each K/V byte is read once for the whole GQA group;
//  - q.k is a matrix product on the matrix cores: 32 tokens at a time,
//    v_mfma_f32_16x16x32_bf16 with K rows (tokens) as the A operand loaded
//    straight from the pool in 16-byte vectors and the queries (from LDS)
//    as B, so no cross-lane reduction is needed;
//  - p.v is a second MFMA: the probabilities come out of the first one
//    already in the A-operand layout of the second (lane l holds head l%16,
//    tokens 8*(l/16)..+7); V is transposed through LDS into the B layout.
//    Each probability enters as two bf16 values, hi + lo (two MFMAs), so
//    the weights keep about 16 significant bits rather than bf16's 8; the
//    latent body (MLA), whose matrix cores are its busiest unit, takes one;
//  - long sequences are split over gridDim.y (flash-decoding): each split
//    writes (max, sum, unnormalised output) and a combine kernel merges
//    them, so a small batch still fills 256 CUs.
// Five bodies share this math. The staged one (head dims 128 or 64, up to
// 16 query heads per KV head, 16-byte rows, power-of-two pages: every
// Llama/Qwen-style decode) loads each block's rows straight into LDS two
// blocks deep; the pipelined one (the other head dims up to 128 on such
// rows) loads the slots of block i+2 and the K/V rows of block i+1 into
// registers while it computes block i, so a wave never waits on the
// dependent slot -> row loads; the latent one (MLA: K rows up to 576 dims, V rows of 512) loads each block
// straight into LDS once for up to 128 heads; the wide one (other shapes
// with many query heads per KV head) stages each block once in LDS for up
// to 64 heads; the generic one serves every other shape (odd dims,
// unaligned rows) one block at a time.
// Metadata errors set the device error word (SGLKV_FLAG_ATTN_*) and skip
// the query, as the reference's kernel does.

typedef __bf16 sglkv_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sglkv_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short sglkv_u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short sglkv_u16x4 __attribute__((ext_vector_type(4)));

namespace {

__device__ __forceinline__ sglkv_bf16x8 attn_as_bf16(sglkv_u16x8 v) {
    return __builtin_bit_cast(sglkv_bf16x8, v);
}

// Eight consecutive bf16 elements [dim, dim + 8) of a K or V head row,
// zero where dim + e >= limit or the token is invalid. VEC: dim and limit
// are multiples of 8 and the row is 16-byte aligned (one 16-byte load).
template <bool VEC>
__device__ __forceinline__ sglkv_u16x8 attn_load8(uint64_t row, uint32_t dim, uint32_t limit,
                                                  bool valid) {
    sglkv_u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (VEC) {
        if (valid && dim < limit)
            v = *reinterpret_cast<__attribute__((address_space(1))) const sglkv_u16x8 *>(row + 2ull * dim);
    } else {
        // Branch- and compare-free: an element past the row (or of an
        // invalid token) loads the row's element 0 and is masked to zero.
        // The caller's row always addresses pool memory (an invalid token's
        // row is slot 0's), so the load stays in bounds. The masks are
        // vector values: (i - limit) >> 31 (arithmetic) is all ones exactly
        // when i < limit (both below 2^31); a compare per element would keep
        // a 64-bit lane mask per load alive in scalar registers until its
        // data returns, more than the SGPR file holds.
        const __attribute__((address_space(1))) uint16_t *p =
            reinterpret_cast<__attribute__((address_space(1))) const uint16_t *>(row);
        const uint32_t vm = valid ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) {
            const uint32_t i = dim + e;
            const uint32_t keep = static_cast<uint32_t>(static_cast<int32_t>(i - limit) >> 31) & vm;
            v[e] = static_cast<uint16_t>(p[i & keep] & keep);
        }
    }
    return v;
}

__device__ __forceinline__ uint16_t attn_to_bf16(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}

// A softmax weight as the sum of two bf16 values, hi = RN(x) and
// lo = RN(x - hi): x - hi is exact in fp32 (|x - hi| <= 2^-8 |x|, at most
// 16 significant bits), so |x - (hi + lo)| <= 2^-16 |x|. The p.v products
// take hi.v + lo.v (two MFMAs into one fp32 accumulator), which keeps the
// weights' error near fp32's instead of bf16's 2^-8; the reference weights
// its values in fp32 (cuda_attention.rs:140-149).
// Element i of the hi and lo operand vectors.
__device__ __forceinline__ void attn_split_bf16(float x, sglkv_u16x8 &hi, sglkv_u16x8 &lo, uint32_t i) {
    const __bf16 h = static_cast<__bf16>(x);
    hi[i] = __builtin_bit_cast(uint16_t, h);
    lo[i] = attn_to_bf16(x - static_cast<float>(h));
}

// Query-level metadata checks of the reference kernel (cuda_attention.rs:
// 59-82). Returns false (and raises the flag once per query) on failure.
__device__ __forceinline__ bool attn_metadata(const sglkv_attn_params &p, uint64_t q, bool report,
                                              uint64_t *start, uint64_t *len) {
    const uint32_t req = p.query_request_indices[q];
    if (req >= p.request_count) {
        if (report) atomicOr(p.flag, SGLKV_FLAG_ATTN_REQUEST);
        return false;
    }
    const uint64_t s = p.request_slot_offsets[req], e = p.request_slot_offsets[req + 1];
    const uint64_t n = p.query_sequence_lengths[q];
    // The launch covers splits * chunk_tokens tokens per query (sized from
    // the caller's maximum length); a longer query is rejected rather than
    // truncated, and the combine pass never reads past its split records.
    if (s > e || e > p.sequence_slot_count || n == 0 || n > e - s ||
        n > p.chunk_tokens * static_cast<uint64_t>(p.splits)) {
        if (report) atomicOr(p.flag, SGLKV_FLAG_ATTN_SEQUENCE);
        return false;
    }
    *start = s;
    *len = n;
    return true;
}

// The work item of this workgroup: query q, KV head kvh, query heads
// [h0, h0 + nh), value dims from d0, tokens [t0, t1) of the sequence that
// starts at sequence_slots[start].
struct attn_work {
    uint64_t q, start, t0, t1;
    uint32_t kvh, h0, nh, d0, split;
    uint32_t dblk;
};

__device__ __forceinline__ bool attn_decode(const sglkv_attn_params &p, uint32_t lane, attn_work *w) {
    // The KV head varies slowest: workgroups are dispatched round-robin
    // over the 8 XCDs, so (with query_count * head_groups * dv_blocks a
    // multiple of 8) every KV head of a query runs on one XCD, and the
    // slices of one token row meet in one L2 rather than eight.
    uint64_t bx = blockIdx.x;
    const uint32_t dblk = static_cast<uint32_t>(bx % p.dv_blocks);
    bx /= p.dv_blocks;
    const uint32_t hg = static_cast<uint32_t>(bx % p.head_groups);
    bx /= p.head_groups;
    const uint64_t q = bx % p.query_count;
    const uint32_t kvh = static_cast<uint32_t>(bx / p.query_count);
    const uint32_t split = blockIdx.y;

    uint64_t start = 0, len = 0;
    const bool report = lane == 0 && split == 0 && hg == 0 && dblk == 0 && kvh == 0;
    if (!attn_metadata(p, q, report, &start, &len)) return false;
    const uint64_t t0 = static_cast<uint64_t>(split) * p.chunk_tokens;
    if (t0 >= len) return false;
    w->q = q;
    w->start = start;
    w->t0 = t0;
    w->t1 = len < t0 + p.chunk_tokens ? len : t0 + p.chunk_tokens;
    w->kvh = kvh;
    w->h0 = kvh * p.group + hg * SGLKV_ATTN_HEADS;
    w->nh = p.group - hg * SGLKV_ATTN_HEADS < SGLKV_ATTN_HEADS ? p.group - hg * SGLKV_ATTN_HEADS
                                                                : SGLKV_ATTN_HEADS;
    w->d0 = dblk * SGLKV_ATTN_DV;
    w->split = split;
    w->dblk = dblk;
    return true;
}

// Queries of the head group into LDS, zero-padded to 16 heads x dk_pad
// dims; a row is dk_pad + 8 elements so the 16 rows start in different
// banks.
__device__ __forceinline__ void attn_stage_queries(const sglkv_attn_params &p, const attn_work &w,
                                                   uint32_t lane, uint16_t *qs, uint32_t qstride) {
    for (uint32_t i = lane; i < SGLKV_ATTN_HEADS * p.dk_pad; i += 64) {
        const uint32_t h = i / p.dk_pad, d = i % p.dk_pad;
        uint16_t v = 0;
        if (h < w.nh && d < p.dk) v = p.queries[(w.q * p.query_heads + w.h0 + h) * p.dk + d];
        qs[h * qstride + d] = v;
    }
    __syncthreads();
}

// Online-softmax state of one wave: lane (g, r) tracks head r.
// NJ = blocks of 16 value dims the wave accumulates.
template <int NJ>
struct attn_state_n {
    float m_run;   // running max (log2 units) of head r
    float l_part;  // this lane's share of head r's sum
    sglkv_f32x4 o[NJ];
};
typedef attn_state_n<SGLKV_ATTN_DV / 16> attn_state;

template <int NJ>
__device__ __forceinline__ void attn_state_init(attn_state_n<NJ> &st) {
    st.m_run = -3.402823466e+38f;
    st.l_part = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < NJ; ++j) st.o[j] = sglkv_f32x4{0.f, 0.f, 0.f, 0.f};
}

// One 32-token block after q.k: sc[b][e] is head r's score of row 4g+e of
// score block b, the token that vt holds at position 8g + 4b + e; vb0/vb1
// the validity ballots of the rows, and vt the block's values transposed
// in LDS (vt[dim][position]). Updates the softmax state and o += p.v.
// vt rows are VTS elements apart.
template <bool FULL_DV = false, int NJ = SGLKV_ATTN_DV / 16, int VTS = SGLKV_ATTN_VT_STRIDE>
__device__ __forceinline__ void attn_softmax_pv(const sglkv_attn_params &p, uint32_t g, uint32_t d0,
                                                const sglkv_f32x4 (&sc)[2], uint64_t vb0, uint64_t vb1,
                                                const uint16_t *vt, uint32_t r, attn_state_n<NJ> &st) {
    float x[8];
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t b = 0; b < 2; ++b)
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) {
            const bool ok = (((b ? vb1 : vb0) >> (4 * g + e)) & 1) != 0;
            const float v = ok ? sc[b][e] * p.scale_log2 : -INFINITY;
            x[4 * b + e] = v;
            mx = fmaxf(mx, v);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(st.m_run, mx);
    const float alpha = exp2f(st.m_run - m_new);
    sglkv_u16x8 phi, plo;
    float psum = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        const float pi = exp2f(x[i] - m_new);
        psum += pi;
        attn_split_bf16(pi, phi, plo, i);
    }
    st.l_part = st.l_part * alpha + psum;
    st.m_run = m_new;

    // Output rows are heads 4g+e: fetch their rescale factors.
    float arow[4];
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) arow[e] = __shfl(alpha, 4 * g + e);
#pragma unroll
    for (uint32_t j = 0; j < NJ; ++j)
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) st.o[j][e] *= arow[e];

    __builtin_amdgcn_wave_barrier();
    // o[head 4g+e][dim 16j + r] += sum_t p[head][t] * v[t][dim], p = hi + lo.
#pragma unroll
    for (uint32_t j = 0; j < NJ; ++j) {
        if (!FULL_DV && d0 + 16 * j >= p.dv) break;
        const sglkv_u16x8 vv = *reinterpret_cast<const sglkv_u16x8 *>(vt + (16 * j + r) * VTS + 8 * g);
        st.o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(phi), attn_as_bf16(vv), st.o[j], 0, 0, 0);
        st.o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(plo), attn_as_bf16(vv), st.o[j], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
}

// Split record i = (q * query_heads + head) * splits + split: its o row
// (SGLKV_ATTN_OPAD floats, 128-byte aligned) and its m, l pair. Records
// are written with non-temporal stores: every workgroup writes its records
// at its end, and streamed out so they do not pile up in L2 (measured on
// the MLA decode: 12.5 us less per launch of the latent body, 1.4 us more
// in the combine that reads them).
__device__ __forceinline__ float *attn_rec_o(const sglkv_attn_params &p, uint64_t i) {
    return p.partial + i * SGLKV_ATTN_OPAD(p.dv);
}
__device__ __forceinline__ float *attn_rec_ml(const sglkv_attn_params &p, uint64_t i) {
    return p.partial + p.query_count * p.query_heads * p.splits * SGLKV_ATTN_OPAD(p.dv) + 2 * i;
}
// The latent body's scaled fp16 records: y row and (m, l, a, 0) of record i.
__device__ __forceinline__ uint16_t *attn_rec_y(const sglkv_attn_params &p, uint64_t i) {
    return reinterpret_cast<uint16_t *>(p.partial) + i * SGLKV_ATTN_HPAD(p.dv);
}
// (m, l, a, 0) of (query q, split, head): ordered by (q, split, head), so
// the heads of one workgroup's split are adjacent and go out in one store.
__device__ __forceinline__ float *attn_rec_mla(const sglkv_attn_params &p, uint64_t q, uint32_t split,
                                               uint64_t head) {
    return reinterpret_cast<float *>(reinterpret_cast<uint16_t *>(p.partial) +
                                     p.query_count * p.query_heads * p.splits * SGLKV_ATTN_HPAD(p.dv)) +
           4 * ((q * p.splits + split) * p.query_heads + head);
}

// Output (one split) or the split record (m, l, o[0..dv)).
template <int NJ>
__device__ __forceinline__ void attn_finish(const sglkv_attn_params &p, const attn_work &w, uint32_t g,
                                            uint32_t r, const attn_state_n<NJ> &st) {
    float l_tot = st.l_part + __shfl_xor(st.l_part, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (p.splits == 1) {
        float linv[4];
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) linv[e] = 1.0f / __shfl(l_tot, 4 * g + e);
#pragma unroll
        for (uint32_t j = 0; j < NJ; ++j) {
            const uint32_t dim = w.d0 + 16 * j + r;
            if (dim >= p.dv) continue;
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) {
                const uint32_t h = 4 * g + e;
                if (h < w.nh)
                    p.output[(w.q * p.query_heads + w.h0 + h) * p.dv + dim] = attn_to_bf16(st.o[j][e] * linv[e]);
            }
        }
    } else {
        if (w.dblk == 0 && g == 0 && r < w.nh) {
            float *pr = attn_rec_ml(p, (w.q * p.query_heads + w.h0 + r) * p.splits + w.split);
            __builtin_nontemporal_store(st.m_run, pr);
            __builtin_nontemporal_store(l_tot, pr + 1);
        }
#pragma unroll
        for (uint32_t j = 0; j < NJ; ++j) {
            const uint32_t dim = w.d0 + 16 * j + r;
            if (dim >= p.dv) continue;
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) {
                const uint32_t h = 4 * g + e;
                if (h < w.nh)
                    __builtin_nontemporal_store(
                        st.o[j][e], attn_rec_o(p, (w.q * p.query_heads + w.h0 + h) * p.splits + w.split) + dim);
            }
        }
    }
}

// Page and in-page position of a slot: shift and mask when the page size
// is a power of two (page_shift < 32), a division otherwise.
__device__ __forceinline__ void attn_split_slot(const sglkv_attn_params &p, uint64_t slot, uint64_t *page,
                                                uint64_t *pos) {
    if (p.page_shift < 32) {
        *page = slot >> p.page_shift;
        *pos = slot & ((1ull << p.page_shift) - 1);
    } else {
        *page = slot / p.page_size;
        *pos = slot % p.page_size;
    }
}

template <bool VEC>
__device__ __forceinline__ void attn_body(const sglkv_attn_params &p) {
    extern __shared__ __attribute__((aligned(16))) uint16_t attn_lds[];
    const uint32_t lane = threadIdx.x;
    const uint32_t g = lane >> 4, r = lane & 15;
    attn_work w;
    if (!attn_decode(p, lane, &w)) return;
    const uint32_t qstride = p.dk_pad + 8;
    uint16_t *qs = attn_lds;
    uint16_t *vt = attn_lds + SGLKV_ATTN_HEADS * qstride;
    attn_stage_queries(p, w, lane, qs, qstride);

    const uint64_t pool = reinterpret_cast<uint64_t>(p.pool);
    const uint64_t kbase = pool + p.key_offset + w.kvh * p.key_head_stride;
    const uint64_t vbase = pool + p.value_offset + w.kvh * p.value_head_stride;
    attn_state st;
    attn_state_init(st);

    for (uint64_t tb = w.t0; tb < w.t1; tb += SGLKV_ATTN_TOKENS) {
        // Row r of score block b is token tb + 8*(r/4) + 4*b + r%4, so that
        // after the q.k product lane (g, r) holds tokens tb + 8g .. 8g+7 of
        // head r: the A-operand layout of the p.v product.
        uint64_t krow[2], vrow[2];
        bool valid[2];
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b) {
            const uint64_t tok = tb + 8 * (r >> 2) + 4 * b + (r & 3);
            bool ok = tok < w.t1;
            uint64_t slot = 0;
            if (ok) {
                slot = p.sequence_slots[w.start + tok];
                if (slot >= p.slot_count) {
                    atomicOr(p.flag, SGLKV_FLAG_ATTN_SLOT);
                    ok = false;
                    slot = 0;
                }
            }
            uint64_t page, pos;
            attn_split_slot(p, slot, &page, &pos);
            krow[b] = kbase + page * p.page_stride + pos * p.key_token_stride;
            vrow[b] = vbase + page * p.page_stride + pos * p.value_token_stride;
            valid[b] = ok;
        }
        // Lane (g, r) loads value dims d0 + 8*(g + 4s) .. +7 of its two
        // tokens. 16-byte pieces are issued first, so their loads are in
        // flight during q.k; element-wise pieces (64 separate 2-byte loads)
        // after it, where they do not hold registers across the q.k loop.
        sglkv_u16x8 vpiece[2][4];
        if (VEC) {
#pragma unroll
            for (uint32_t b = 0; b < 2; ++b)
#pragma unroll
                for (uint32_t s = 0; s < 4; ++s)
                    vpiece[b][s] = attn_load8<VEC>(vrow[b], w.d0 + 8 * (g + 4 * s), p.dv, valid[b]);
        }

        // Scores: s[b][e] = q(head r) . k(token of row 4g+e of block b).
        sglkv_f32x4 sc[2] = {sglkv_f32x4{0.f, 0.f, 0.f, 0.f}, sglkv_f32x4{0.f, 0.f, 0.f, 0.f}};
        for (uint32_t kk = 0; kk < p.dk_pad; kk += 32) {
            const sglkv_u16x8 qv = *reinterpret_cast<const sglkv_u16x8 *>(qs + r * qstride + kk + 8 * g);
#pragma unroll
            for (uint32_t b = 0; b < 2; ++b) {
                const sglkv_u16x8 kv = attn_load8<VEC>(krow[b], kk + 8 * g, p.dk, valid[b]);
                sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(kv), attn_as_bf16(qv), sc[b],
                                                                0, 0, 0);
            }
        }

        if (!VEC) {
#pragma unroll
            for (uint32_t b = 0; b < 2; ++b)
#pragma unroll
                for (uint32_t s = 0; s < 4; ++s)
                    vpiece[b][s] = attn_load8<VEC>(vrow[b], w.d0 + 8 * (g + 4 * s), p.dv, valid[b]);
        }
        // Transposed values into LDS: vt[dim][token - tb].
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b) {
            const uint32_t tl = 8 * (r >> 2) + 4 * b + (r & 3);
#pragma unroll
            for (uint32_t s = 0; s < 4; ++s)
#pragma unroll
                for (uint32_t e = 0; e < 8; ++e)
                    vt[(8 * (g + 4 * s) + e) * SGLKV_ATTN_VT_STRIDE + tl] = vpiece[b][s][e];
        }
        const uint64_t vb0 = __ballot(valid[0]), vb1 = __ballot(valid[1]);
        attn_softmax_pv(p, g, w.d0, sc, vb0, vb1, vt, r, st);
    }
    attn_finish(p, w, g, r, st);
}

// ---- Pipelined body: head dims <= 128 on 16-byte rows --------------------
//
// The host sends shapes here only when every row is 16-byte aligned, dk and
// dv are at most 128, the page size is a power of two and page and token
// strides fit 32 bits (and slot_count < 2^32). Per 32-token block a lane
// needs six slots: K rows
// kr(b) = 8*(r/4) + 4b + r%4 (b = 0, 1; the q.k A-operand rows, as in the
// generic body) and V rows 4*tg + i (i = 0..3, tg = lane % 8), whose dims
// 16*dg .. +15 (dg = lane / 8) it loads as two 16-byte pieces; four
// consecutive tokens of a dim then go to LDS as one 8-byte store.
//
// The loop keeps two blocks of rows in flight: block i+1's rows and block
// i+2's slots are issued before block i is computed, slots first, because
// the memory counter retires loads in issue order (waiting for a slot load
// issued after a row load would wait for the row load too). Every load is
// unconditional: a row past the end of the chunk, or whose slot is outside
// the pool, reads the context's zero row instead, so the compiler can
// count the loads in flight exactly and padded tokens contribute exact
// zeros (never garbage) to p.v.
// Slots of one block: lane l holds the raw slot of token l % 32 (lanes
// 32..63 repeat lanes 0..31), one 8-byte load per lane.
struct attn_pipe_slots {
    uint64_t raw;
};

struct attn_pipe_rows {
    sglkv_u16x8 k[8];  // k[4b + c]: K row kr(b), dims 32c + 8g .. +7
    sglkv_u16x8 v[8];  // v[2i + h]: V row 4tg + i, dims 16dg + 8h .. +7
    uint32_t kvalid;   // bit b: K row kr(b) valid
};

__device__ __forceinline__ uint32_t attn_pipe_row(uint32_t j, uint32_t r, uint32_t tg) {
    return j < 2 ? 8 * (r >> 2) + 4 * j + (r & 3) : 4 * tg + (j - 2);
}

__device__ __forceinline__ void attn_pipe_load_slots(const sglkv_attn_params &p, const attn_work &w,
                                                     uint64_t tb, uint32_t lane, attn_pipe_slots &sl) {
    uint64_t tok = tb + (lane & 31);
    tok = tok < w.t1 ? tok : w.t1 - 1;  // in range; validity is decided at use
    sl.raw = p.sequence_slots[w.start + tok];
}

// 16 bytes at `row + off`, or at `zero + off` when the piece is masked.
__device__ __forceinline__ sglkv_u16x8 attn_pipe_piece(uint64_t row, uint64_t zero, uint32_t off,
                                                       bool ok) {
    return *reinterpret_cast<__attribute__((address_space(1))) const sglkv_u16x8 *>((ok ? row : zero) + off);
}

// Rows of block tb from its slots: each lane validates the slot it loaded
// (raising the error word for one outside the pool), and the six slots a
// lane needs arrive by cross-lane permutes, which wait on the LDS counter,
// not on the memory counter the row loads are pipelined on.
template <bool FULL>
__device__ __forceinline__ void attn_pipe_load_rows(const sglkv_attn_params &p, const attn_work &w,
                                                    uint64_t tb, uint64_t kbase, uint64_t vbase,
                                                    uint32_t lane, uint32_t g, uint32_t r, uint32_t tg,
                                                    uint32_t dg, const attn_pipe_slots &sl,
                                                    attn_pipe_rows &rw) {
    constexpr uint32_t kInvalid = 0xFFFFFFFFu;  // the host keeps slot_count below 2^32
    const uint64_t zero = reinterpret_cast<uint64_t>(p.zero_row);
    const uint32_t mask = (1u << p.page_shift) - 1;
    uint32_t mine = kInvalid;
    if (tb + (lane & 31) < w.t1) {
        if (sl.raw < p.slot_count)
            mine = static_cast<uint32_t>(sl.raw);
        else
            atomicOr(p.flag, SGLKV_FLAG_ATTN_SLOT);
    }
    rw.kvalid = 0;
#pragma unroll
    for (uint32_t j = 0; j < 6; ++j) {
        const uint32_t s32 = static_cast<uint32_t>(__shfl(static_cast<int>(mine), attn_pipe_row(j, r, tg)));
        const bool ok = s32 != kInvalid;
        const uint32_t page = s32 >> p.page_shift, pos = s32 & mask;
        if (j < 2) {
            const uint64_t row = kbase + static_cast<uint64_t>(page) * p.page_stride32 +
                                 static_cast<uint64_t>(pos) * p.key_token_stride32;
            rw.kvalid |= (ok ? 1u : 0u) << j;
#pragma unroll
            for (uint32_t c = 0; c < 4; ++c) {
                const uint32_t dim = 32 * c + 8 * g;
                rw.k[4 * j + c] = attn_pipe_piece(row, zero, 2 * dim, ok && (FULL || dim < p.dk));
            }
        } else {
            const uint64_t row = vbase + static_cast<uint64_t>(page) * p.page_stride32 +
                                 static_cast<uint64_t>(pos) * p.value_token_stride32;
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h) {
                const uint32_t dim = 16 * dg + 8 * h;
                rw.v[2 * (j - 2) + h] = attn_pipe_piece(row, zero, 2 * dim, ok && (FULL || dim < p.dv));
            }
        }
    }
}

template <bool FULL>
__device__ __forceinline__ void attn_pipe_block(const sglkv_attn_params &p, uint32_t g, uint32_t r,
                                                uint32_t tg, uint32_t dg, const uint16_t *qs,
                                                uint32_t qstride, uint16_t *vt, const attn_pipe_rows &rw,
                                                attn_state &st) {
    // V transposed into LDS, four tokens of one dim per 8-byte store.
#pragma unroll
    for (uint32_t e = 0; e < 16; ++e) {
        sglkv_u16x4 t4;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) t4[i] = rw.v[2 * i + (e >> 3)][e & 7];
        *reinterpret_cast<sglkv_u16x4 *>(vt + (16 * dg + e) * SGLKV_ATTN_VT_STRIDE + 4 * tg) = t4;
    }
    sglkv_f32x4 sc[2] = {sglkv_f32x4{0.f, 0.f, 0.f, 0.f}, sglkv_f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
        if (!FULL && 32 * c >= p.dk_pad) break;
        const sglkv_u16x8 qv = *reinterpret_cast<const sglkv_u16x8 *>(qs + r * qstride + 32 * c + 8 * g);
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b)
            sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(rw.k[4 * b + c]), attn_as_bf16(qv),
                                                            sc[b], 0, 0, 0);
    }
    const uint64_t vb0 = __ballot(rw.kvalid & 1), vb1 = __ballot((rw.kvalid >> 1) & 1);
    attn_softmax_pv<FULL>(p, g, 0, sc, vb0, vb1, vt, r, st);
}

#ifndef SGLKV_ATTN_PIPE_DEPTH
#define SGLKV_ATTN_PIPE_DEPTH 2  /* blocks of rows per wave: one computing, the rest in flight (even) */
#endif

template <bool FULL>
__device__ __forceinline__ void attn_pipe_body(const sglkv_attn_params &p) {
    constexpr uint32_t N = SGLKV_ATTN_PIPE_DEPTH;
    static_assert(N >= 2 && N % 2 == 0, "the slot buffers alternate by block parity");
    extern __shared__ __attribute__((aligned(16))) uint16_t attn_lds[];
    const uint32_t lane = threadIdx.x;
    const uint32_t g = lane >> 4, r = lane & 15;
    const uint32_t tg = lane & 7, dg = lane >> 3;
    attn_work w;
    if (!attn_decode(p, lane, &w)) return;
    const uint32_t qstride = p.dk_pad + 8;
    uint16_t *qs = attn_lds;
    uint16_t *vt = attn_lds + SGLKV_ATTN_HEADS * qstride;

    const uint64_t pool = reinterpret_cast<uint64_t>(p.pool);
    const uint64_t kbase = pool + p.key_offset + w.kvh * p.key_head_stride;
    const uint64_t vbase = pool + p.value_offset + w.kvh * p.value_head_stride;
    constexpr uint32_t B = SGLKV_ATTN_TOKENS;
    attn_state st;
    attn_state_init(st);

    // Block k (tokens t0 + k*B ..) has its slots in sl[k % 2] and its rows
    // in rw[k % N]. Prologue: rows of blocks 0 .. N-2, slots of block N-1.
    // The prologue issues in the loop's order (the slots of block k+1
    // before the rows of block k), so the loads in flight on entering the
    // loop match those at the end of a trip and the compiler's wait counts
    // stay exact across the back edge.
    attn_pipe_slots sl[2];
    attn_pipe_rows rw[N];
    attn_pipe_load_slots(p, w, w.t0, lane, sl[0]);
    // The queries are staged while the first slots are in flight.
    attn_stage_queries(p, w, lane, qs, qstride);
#pragma unroll
    for (uint32_t k = 0; k + 1 < N; ++k) {
        attn_pipe_load_slots(p, w, w.t0 + (k + 1) * B, lane, sl[(k + 1) % 2]);
        __builtin_amdgcn_sched_barrier(0);  // keep the issue order: slots, then rows
        attn_pipe_load_rows<FULL>(p, w, w.t0 + k * B, kbase, vbase, lane, g, r, tg, dg, sl[k % 2], rw[k]);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Steady state, N blocks per trip so every buffer index is a constant:
    // at block k, load the slots of block k+N, then the rows of block
    // k+N-1, then compute block k.
    for (uint64_t tb = w.t0;; tb += N * B) {
        bool done = false;
#pragma unroll
        for (uint32_t u = 0; u < N; ++u) {
            const uint64_t t = tb + u * B;
            attn_pipe_load_slots(p, w, t + N * B, lane, sl[u % 2]);
            __builtin_amdgcn_sched_barrier(0);
            attn_pipe_load_rows<FULL>(p, w, t + (N - 1) * B, kbase, vbase, lane, g, r, tg, dg,
                                      sl[(u + 1) % 2], rw[(u + N - 1) % N]);
            __builtin_amdgcn_sched_barrier(0);
            attn_pipe_block<FULL>(p, g, r, tg, dg, qs, qstride, vt, rw[u], st);
            if (t + B >= w.t1) {
                done = true;
                break;
            }
        }
        if (done) break;
    }
    attn_finish(p, w, g, r, st);
}

// ---- Wide body: many query heads per KV head (MLA), dims up to 576/512 ----
//
// The reference's MLA decode calls this attention with every query head of
// the model over one latent KV head (crates/sglang-srt/src/cuda_mla.rs:
// 273-294): 128 heads, K rows of 576 and V rows of 512 for DeepSeek-V3.
// Per-wave bodies would read each K row once per 16-head group and per
// 128-dim value block (32 times for that shape). Here a workgroup of eight
// waves owns (query, KV head, up to 4 groups of 16 query heads) and stages
// each 32-token block once in LDS, row-major as the pool holds it. The two
// waves of a head group share one SIMD and split the work in halves: wave
// (group, half) computes q.k over key dims [half, half + 1) * dk/2 with that
// half of the queries in registers, the two partial score tiles meet
// through LDS (each wave adds the other's to its own, so both hold the
// same scores), and each accumulates p.v for its half of the value dims.
// Nothing is computed twice, and a wave holds 16 heads x dv/2 outputs.
//
// Rows stay in flight from HBM across the loop, in registers. Iteration k
// (block k's K rows in LDS): issue block k+2's K rows into one register
// stage between the q.k MFMAs of block k, write block k's V rows (loaded
// during the previous iteration) to LDS and issue block k+1's V rows,
// barrier; write block k+1's K rows (the other stage, loaded an iteration
// earlier) between the p.v MFMAs of block k, barrier. One LDS stage serves:
// K rows are only read by q.k and V rows only by p.v, and the two barriers
// keep each area's writers and readers apart. The chunk's slots are read,
// checked and kept in an LDS table at the start.
//
// q.k: score block b covers tokens 16b .. 16b+15, so lane (g, r) holds head
// r's scores of tokens 16b + 4g + e. p.v takes those as k index 8g + 4b + e;
// its B operand (V[token][dim]) comes from two transposing LDS reads
// (ds_read_b64_tr_b16: within 16 lanes, lane j's element i is element j%4
// of the 8 bytes addressed by lane 4i + j/4), lane r of group g pointing at
// row 4g + r/4 (then 16 + 4g + r/4), dims 4(r%4) of the 16-dim block.
//
// Softmax reference: the first valid block of a split fixes head h's
// reference maximum m, and every later block adds p = 2^(x - m) without
// rescaling, so nothing but MFMAs touches the accumulators in the loop. The
// split record carries (m, l, o) relative to that reference, which is what
// the combine pass needs of it. That is exact arithmetic as long as p stays
// representable: a block whose maximum exceeds m by more than
// SGLKV_ATTN_FIXED_MAX_LOG2 flags the workgroup, which then recomputes its
// split with the usual per-block rescaling. With the bound at 64 and chunks
// of at most SGLKV_ATTN_WIDE_SLOTS tokens, l < 2^76 and o stays finite for
// |v| < 4e15.

#define SGLKV_ATTN_FIXED_MAX_LOG2 64.0f

template <int DKC, int NJ>  // K dims padded to 32*DKC, V dims to 16*NJ (both even)
struct attn_wide_geom {
    static constexpr uint32_t B = SGLKV_ATTN_TOKENS;
    static constexpr uint32_t WAVES = SGLKV_ATTN_WIDE_WAVES;
    static constexpr uint32_t GROUPS = SGLKV_ATTN_WIDE_GROUPS;
    static constexpr uint32_t THREADS = 64 * WAVES;
    static constexpr uint32_t KH = DKC / 2;        // q.k k-steps of one wave
    static constexpr uint32_t NJH = NJ / 2;        // value blocks of one wave
    static constexpr uint32_t KS = 32 * DKC + 8;   // LDS K row stride (u16)
    static constexpr uint32_t VS = 16 * NJ + 16;   // LDS V row stride (u16)
    static constexpr uint32_t KCOLS = 4 * DKC;     // 16-byte pieces per K row
    static constexpr uint32_t VCOLS = 2 * NJ;      // 16-byte pieces per V row
    // Thread t moves column t % COLS of tokens (t / COLS) * PT + i, i < PT:
    // K columns [0, KM) and every V column that way; the KR columns past KM
    // (576-wide keys: 8) are one piece of threads t < B * KR, token t / KR.
    // A thread's tokens are consecutive, so their slots come in one read.
    static constexpr uint32_t KM = KCOLS < 64 ? KCOLS : 64;
    static constexpr uint32_t KR = KCOLS - KM;
    static constexpr uint32_t KPT = B * KM / THREADS;
    static constexpr uint32_t VPT = B * VCOLS / THREADS;
    static constexpr uint32_t RTHREADS = B * KR;
    static constexpr uint32_t KS_ELEMS = B * KS;
    static constexpr uint32_t VS_ELEMS = B * VS;
    static constexpr uint32_t SX_BYTES = WAVES * 2 * 64 * 16;  // partial score tiles
    static constexpr uint32_t LDS_BYTES = 2 * (KS_ELEMS + VS_ELEMS) + SX_BYTES + 4 * SGLKV_ATTN_WIDE_SLOTS + 16;
    static constexpr uint32_t QK_AHEAD = KH < 2 ? KH : 2;    // LDS reads issued ahead of their MFMAs
    static constexpr uint32_t PV_AHEAD = NJH < 2 ? NJH : 2;
    static_assert(DKC % 2 == 0 && NJ % 2 == 0 && DKC <= 18 && NJ <= 32, "halves of one head group");
    static_assert(WAVES == 2 * GROUPS, "two waves per head group");
    static_assert(THREADS % KM == 0 && THREADS % VCOLS == 0 && KPT >= 1 && VPT >= 1, "whole rows per pass");
    static_assert(RTHREADS <= THREADS, "one remainder piece per thread at most");
    static_assert(LDS_BYTES == SGLKV_ATTN_WIDE_LDS_BYTES(DKC, NJ), "the host sizes the same LDS");
    static_assert(SGLKV_ATTN_WIDE_SLOTS % B == 0, "whole blocks in the slot table");
};

constexpr uint32_t kAttnInvalidSlot = 0xFFFFFFFFu;  // the host keeps slot_count below 2^32

// A slot value of token `tok` checked against the chunk end and the pool.
__device__ __forceinline__ uint32_t attn_wide_slot(const sglkv_attn_params &p, uint64_t raw, uint64_t tok,
                                                   uint64_t t1) {
    if (tok >= t1) return kAttnInvalidSlot;
    if (raw >= p.slot_count) {
        atomicOr(p.flag, SGLKV_FLAG_ATTN_SLOT);
        return kAttnInvalidSlot;
    }
    return static_cast<uint32_t>(raw);
}

// One thread's share of a block (the pieces named in attn_wide_geom); the
// main loop keeps two of these for K rows and uses one's v for V rows.
template <int DKC, int NJ>
struct attn_wide_stage {
    sglkv_u16x8 k[attn_wide_geom<DKC, NJ>::KPT];
    sglkv_u16x8 v[attn_wide_geom<DKC, NJ>::VPT];
    sglkv_u16x8 kr;
};

// 16 bytes at base + (row of slot s32) + off, or at the zero row when !ok:
// the row offset is masked and the base selected, so the address is pure
// arithmetic (no branch around the load).
__device__ __forceinline__ sglkv_u16x8 attn_wide_get(const sglkv_attn_params &p, uint64_t base, uint32_t s32,
                                                     uint32_t stride, uint32_t off, bool ok) {
    const uint64_t row = static_cast<uint64_t>(s32 >> p.page_shift) * p.page_stride32 +
                         static_cast<uint64_t>(s32 & ((1u << p.page_shift) - 1)) * stride + off;
    const uint64_t at = (ok ? base : reinterpret_cast<uint64_t>(p.zero_row)) + (row & (ok ? ~0ull : 0ull));
    return *reinterpret_cast<__attribute__((address_space(1))) const sglkv_u16x8 *>(at);
}

// N consecutive slots from the LDS table (16-byte aligned when N % 4 == 0).
template <uint32_t N>
__device__ __forceinline__ void attn_wide_slots(const uint32_t *at, uint32_t (&s)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (uint32_t i = 0; i < N; i += 4) {
            const uint4 v = *reinterpret_cast<const uint4 *>(at + i);
            s[i] = v.x, s[i + 1] = v.y, s[i + 2] = v.z, s[i + 3] = v.w;
        }
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (uint32_t i = 0; i < N; i += 2) {
            const uint2 v = *reinterpret_cast<const uint2 *>(at + i);
            s[i] = v.x, s[i + 1] = v.y;
        }
    } else {
#pragma unroll
        for (uint32_t i = 0; i < N; ++i) s[i] = at[i];
    }
}

// Issues the loads of the K rows (attn_wide_load_k) or V rows
// (attn_wide_load_v) of the block whose slots start at `slots`; a piece of
// an invalid token or past dk / dv reads the zero row.
template <int DKC, int NJ>
__device__ __forceinline__ void attn_wide_load_k(const sglkv_attn_params &p, uint64_t kbase, const uint32_t *slots,
                                                 uint32_t tid, attn_wide_stage<DKC, NJ> &st) {
    typedef attn_wide_geom<DKC, NJ> G;
    uint32_t sk[G::KPT];
    attn_wide_slots(slots + (tid / G::KM) * G::KPT, sk);
    const bool rem = G::RTHREADS != 0 && tid < G::RTHREADS;
    const uint32_t rcol = G::KM + tid % (G::KR ? G::KR : 1);
    const uint32_t sr = rem ? slots[tid / (G::KR ? G::KR : 1)] : kAttnInvalidSlot;
    const uint32_t col = tid % G::KM;
    const bool in = 8 * col < p.dk;
#pragma unroll
    for (uint32_t i = 0; i < G::KPT; ++i)
        st.k[i] = attn_wide_get(p, kbase, sk[i], p.key_token_stride32, 16 * col, in && sk[i] != kAttnInvalidSlot);
    if (G::RTHREADS != 0)
        st.kr = attn_wide_get(p, kbase, sr, p.key_token_stride32, 16 * rcol,
                              rem && 8 * rcol < p.dk && sr != kAttnInvalidSlot);
}

template <int DKC, int NJ>
__device__ __forceinline__ void attn_wide_load_v(const sglkv_attn_params &p, uint64_t vbase, const uint32_t *slots,
                                                 uint32_t tid, attn_wide_stage<DKC, NJ> &st) {
    typedef attn_wide_geom<DKC, NJ> G;
    uint32_t sv[G::VPT];
    attn_wide_slots(slots + (tid / G::VCOLS) * G::VPT, sv);
    const uint32_t col = tid % G::VCOLS;
    const bool in = 8 * col < p.dv;
#pragma unroll
    for (uint32_t i = 0; i < G::VPT; ++i)
        st.v[i] = attn_wide_get(p, vbase, sv[i], p.value_token_stride32, 16 * col, in && sv[i] != kAttnInvalidSlot);
}

template <int DKC, int NJ>
__device__ __forceinline__ void attn_wide_store_k(uint16_t *ks, uint32_t tid, const attn_wide_stage<DKC, NJ> &st) {
    typedef attn_wide_geom<DKC, NJ> G;
    uint16_t *at = ks + (tid / G::KM) * G::KPT * G::KS + 8 * (tid % G::KM);
#pragma unroll
    for (uint32_t i = 0; i < G::KPT; ++i) *reinterpret_cast<sglkv_u16x8 *>(at + i * G::KS) = st.k[i];
    if (G::RTHREADS != 0 && tid < G::RTHREADS) {
        const uint32_t kr = G::KR ? G::KR : 1;
        *reinterpret_cast<sglkv_u16x8 *>(ks + (tid / kr) * G::KS + 8 * (G::KM + tid % kr)) = st.kr;
    }
}

template <int DKC, int NJ>
__device__ __forceinline__ void attn_wide_store_v(uint16_t *vs, uint32_t tid, const attn_wide_stage<DKC, NJ> &st) {
    typedef attn_wide_geom<DKC, NJ> G;
    uint16_t *at = vs + (tid / G::VCOLS) * G::VPT * G::VS + 8 * (tid % G::VCOLS);
#pragma unroll
    for (uint32_t i = 0; i < G::VPT; ++i) *reinterpret_cast<sglkv_u16x8 *>(at + i * G::VS) = st.v[i];
}

typedef short attn_i16x4 __attribute__((ext_vector_type(4)));

// Four u16 of V for the p.v B operand (see the layout note above).
__device__ __forceinline__ attn_i16x4 attn_wide_vtr(const uint16_t *at) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) attn_i16x4 *)(reinterpret_cast<uintptr_t>(at)));
}

// Scheduling masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedVmemRead = 0x020, kSchedDsRead = 0x100;

// This wave's partial q.k of the staged block over its KH k-steps (queries
// qf), left in sc and written to its score tile (sxw[b * 64 + lane]). PIN:
// the group barriers make the LDS reads run QK_AHEAD k-steps ahead of the
// MFMAs that use them (otherwise the caller pins the whole region).
template <int DKC, int NJ, bool PIN = true>
__device__ __forceinline__ void attn_wide_qk(const uint16_t *ks, const sglkv_u16x8 (&qf)[DKC / 2], uint32_t kc0,
                                             uint32_t g, uint32_t r, uint32_t lane, sglkv_f32x4 (&sc)[2],
                                             sglkv_f32x4 *sxw) {
    typedef attn_wide_geom<DKC, NJ> G;
    const uint16_t *k0 = ks + r * G::KS + 32 * kc0 + 8 * g, *k1 = k0 + 16 * G::KS;
    sglkv_u16x8 kf[G::KH][2];
#pragma unroll
    for (uint32_t c = 0; c < G::KH; ++c) {
        kf[c][0] = *reinterpret_cast<const sglkv_u16x8 *>(k0 + 32 * c);
        kf[c][1] = *reinterpret_cast<const sglkv_u16x8 *>(k1 + 32 * c);
    }
    sc[0] = sc[1] = sglkv_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t c = 0; c < G::KH; ++c)
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b)
            sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(kf[c][b]), attn_as_bf16(qf[c]), sc[b], 0, 0, 0);
    if (PIN) {
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * G::QK_AHEAD, 0);
#pragma unroll
        for (uint32_t c = 0; c < G::KH - G::QK_AHEAD; ++c) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2 * G::QK_AHEAD, 0);
    }
    sxw[lane] = sc[0];
    sxw[64 + lane] = sc[1];
}

// Adds the other half's partial scores (sxo) to sc, then softmax and p.v
// over this wave's value blocks (from dim 16 * j0). EXACT: the running
// maximum and per-block rescaling; otherwise the fixed reference, with
// *over set when a block exceeds it. PIN as for attn_wide_qk.
template <bool EXACT, int DKC, int NJ, bool PIN = true>
__device__ __forceinline__ void attn_wide_pv(const sglkv_attn_params &p, const uint16_t *vs, sglkv_f32x4 (&sc)[2],
                                             const sglkv_f32x4 *sxo, const uint32_t *cur, uint32_t j0, uint32_t g,
                                             uint32_t r, uint32_t lane, attn_state_n<NJ / 2> &st, bool *over) {
    typedef attn_wide_geom<DKC, NJ> G;
    sc[0] += sxo[lane];
    sc[1] += sxo[64 + lane];
    // Bit 4g+e of ballot b: token 16b + 4g + e is valid.
    const uint64_t vb0 = __ballot(cur[r] != kAttnInvalidSlot);
    const uint64_t vb1 = __ballot(cur[16 + r] != kAttnInvalidSlot);
    float x[8];
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t b = 0; b < 2; ++b)
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) {
            const bool ok = (((b ? vb1 : vb0) >> (4 * g + e)) & 1) != 0;
            const float v = ok ? sc[b][e] * p.scale_log2 : -INFINITY;
            x[4 * b + e] = v;
            mx = fmaxf(mx, v);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    sglkv_u16x8 phi, plo;
    float psum = 0.0f;
    if (EXACT) {
        const float m_new = fmaxf(st.m_run, mx);
        const float alpha = exp2f(st.m_run - m_new);
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const float pi = exp2f(x[i] - m_new);
            psum += pi;
            attn_split_bf16(pi, phi, plo, i);
        }
        st.l_part = st.l_part * alpha + psum;
        st.m_run = m_new;
        float arow[4];
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) arow[e] = __shfl(alpha, 4 * g + e);
#pragma unroll
        for (uint32_t j = 0; j < G::NJH; ++j)
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) st.o[j][e] *= arow[e];
    } else {
        // m_run is -inf until a valid token arrives (l and o are zero until
        // then, so fixing the reference needs no rescale).
        if (st.m_run == -INFINITY) st.m_run = mx;
        const float m_ref = st.m_run == -INFINITY ? 0.0f : st.m_run;
        *over = *over || mx > m_ref + SGLKV_ATTN_FIXED_MAX_LOG2;
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const float pi = exp2f(fminf(x[i] - m_ref, SGLKV_ATTN_FIXED_MAX_LOG2));
            psum += pi;
            attn_split_bf16(pi, phi, plo, i);
        }
        st.l_part += psum;
    }
    // o[head 4g+e][dim 16(j0 + j) + r] += sum over the block of p * v. Every
    // value block is computed: staged dims past dv are zero, and the finish
    // writes none of them.
    const uint16_t *v0 = vs + (4 * g + (r >> 2)) * G::VS + 4 * (r & 3) + 16 * j0;
    if (EXACT) {
        // The exact path runs in a loop of its own (the rare recompute of a
        // split): an opaque base keeps the compiler from hoisting the
        // 2 * NJH read addresses out of that loop into registers it then
        // has to spill; it forms them per block instead.
        uintptr_t a = reinterpret_cast<uintptr_t>(v0);
        asm volatile("" : "+v"(a));
        v0 = reinterpret_cast<const uint16_t *>(a);
    }
    attn_i16x4 vlo[G::NJH], vhi[G::NJH];
#pragma unroll
    for (uint32_t j = 0; j < G::NJH; ++j) {
        vlo[j] = attn_wide_vtr(v0 + 16 * j);
        vhi[j] = attn_wide_vtr(v0 + 16 * G::VS + 16 * j);
    }
#pragma unroll
    for (uint32_t j = 0; j < G::NJH; ++j) {
        const sglkv_u16x8 vv = {(uint16_t)vlo[j][0], (uint16_t)vlo[j][1], (uint16_t)vlo[j][2], (uint16_t)vlo[j][3],
                                (uint16_t)vhi[j][0], (uint16_t)vhi[j][1], (uint16_t)vhi[j][2], (uint16_t)vhi[j][3]};
        st.o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(phi), attn_as_bf16(vv), st.o[j], 0, 0, 0);
        st.o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(plo), attn_as_bf16(vv), st.o[j], 0, 0, 0);
    }
    if (PIN) {
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * G::PV_AHEAD, 1);
#pragma unroll
        for (uint32_t j = 0; j < G::NJH - G::PV_AHEAD; ++j) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 1);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 1);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2 * G::PV_AHEAD, 1);
    }
}

template <int DKC, int NJ>
__device__ __forceinline__ void attn_wide_body(const sglkv_attn_params &p) {
    typedef attn_wide_geom<DKC, NJ> G;
    constexpr uint32_t B = G::B;
    extern __shared__ __attribute__((aligned(16))) uint16_t attn_lds[];
    uint16_t *ks = attn_lds, *vs = attn_lds + G::KS_ELEMS;
    sglkv_f32x4 *sx = reinterpret_cast<sglkv_f32x4 *>(vs + G::VS_ELEMS);           // [wave][b][lane]
    uint32_t *slots = reinterpret_cast<uint32_t *>(vs + G::VS_ELEMS + G::SX_BYTES / 2);
    uint32_t *redo = slots + SGLKV_ATTN_WIDE_SLOTS;  // set: recompute the split exactly
    const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t g = lane >> 4, r = lane & 15;
    const uint32_t grp = wv % G::GROUPS, half = wv / G::GROUPS;
    sglkv_f32x4 *sxw = sx + wv * 128, *sxo = sx + (wv ^ G::GROUPS) * 128;

    // Workgroup -> (query, KV head, block of up to 4 head groups); the head
    // block varies slowest, so the workgroups of one query that read the
    // same rows run on one XCD when query_count * kv_heads is a multiple
    // of 8.
    const uint32_t hblocks = (p.head_groups + G::GROUPS - 1) / G::GROUPS;
    uint64_t bx = blockIdx.x;
    const uint64_t q = bx % p.query_count;
    bx /= p.query_count;
    const uint32_t kvh = static_cast<uint32_t>(bx % p.kv_heads);
    const uint32_t hb = static_cast<uint32_t>(bx / p.kv_heads);
    const uint32_t split = blockIdx.y;
    uint64_t start = 0, len = 0;
    if (!attn_metadata(p, q, tid == 0 && split == 0 && hb == 0 && kvh == 0, &start, &len)) return;
    const uint64_t t0 = static_cast<uint64_t>(split) * p.chunk_tokens;
    if (t0 >= len || hb >= hblocks) return;
    const uint64_t t1 = len < t0 + p.chunk_tokens ? len : t0 + p.chunk_tokens;
    const uint32_t nb = static_cast<uint32_t>((t1 - t0 + B - 1) / B);  // <= SLOTS / B (host bound)
    const uint32_t hg = hb * G::GROUPS + grp;
    const bool active = hg < p.head_groups;  // the same for both waves of a group
    attn_work w;
    w.q = q;
    w.start = start;
    w.t0 = t0;
    w.t1 = t1;
    w.kvh = kvh;
    w.h0 = kvh * p.group + hg * SGLKV_ATTN_HEADS;
    w.nh = !active ? 0
                   : (p.group - hg * SGLKV_ATTN_HEADS < SGLKV_ATTN_HEADS ? p.group - hg * SGLKV_ATTN_HEADS
                                                                         : SGLKV_ATTN_HEADS);
    w.d0 = half * 16 * G::NJH;
    w.split = split;
    w.dblk = half;  // only the first half writes a split record's (m, l)
    const uint32_t kc0 = half * G::KH, j0 = half * G::NJH;

    // This half's queries: lane (g, r) holds head r, dims 32(kc0 + c) + 8g
    // .. +7 (zero past the group or past dk); the host requires 16-byte
    // aligned queries.
    auto load_queries = [&](sglkv_u16x8(&qv)[G::KH]) {
#pragma unroll
        for (uint32_t c = 0; c < G::KH; ++c) {
            const uint32_t d = 32 * (kc0 + c) + 8 * g;
            qv[c] = sglkv_u16x8{0, 0, 0, 0, 0, 0, 0, 0};
            if (r < w.nh && d < p.dk)
                qv[c] = *reinterpret_cast<const sglkv_u16x8 *>(p.queries + (q * p.query_heads + w.h0 + r) * p.dk + d);
        }
    };
    sglkv_u16x8 qf[G::KH];
    load_queries(qf);

    // The chunk's slots, checked once; tokens past t1 are invalid.
    if (tid == 0) *redo = 0;
    for (uint32_t i = tid; i < nb * B; i += G::THREADS) {
        const uint64_t tok = t0 + i;
        slots[i] = attn_wide_slot(p, tok < t1 ? p.sequence_slots[start + tok] : 0, tok, t1);
    }
    __syncthreads();

    const uint64_t pool = reinterpret_cast<uint64_t>(p.pool);
    const uint64_t kbase = pool + p.key_offset + kvh * p.key_head_stride;
    const uint64_t vbase = pool + p.value_offset + kvh * p.value_head_stride;
    // K rows in registers: two stages where the register file has room
    // (block k+2's rows load while block k+1's wait for LDS); one stage for
    // 576-wide keys, where two stages with the 16 value accumulators and the
    // queries would not fit a wave's 256 registers (8 waves per workgroup,
    // two per SIMD): there block k+2's rows load only once block k+1's are
    // in LDS. V rows: ra.v.
    constexpr bool two_stages = DKC < 18;
    attn_wide_stage<DKC, NJ> ra, rb;
    attn_wide_load_k<DKC, NJ>(p, kbase, slots, tid, ra);
    attn_wide_load_v<DKC, NJ>(p, vbase, slots, tid, ra);
    if (two_stages) attn_wide_load_k<DKC, NJ>(p, kbase, slots + (nb > 1 ? B : 0), tid, rb);
    attn_wide_store_k<DKC, NJ>(ks, tid, ra);
    if (!two_stages) attn_wide_load_k<DKC, NJ>(p, kbase, slots + (nb > 1 ? B : 0), tid, ra);
    __syncthreads();

    attn_state_n<G::NJH> st;
    attn_state_init(st);
    st.m_run = -INFINITY;  // reference not fixed yet
    bool over = false;
    // One iteration (block k; `fr` is the K stage block k left, `next`
    // holds block k+1's K rows). Loads and stores run whether or not their
    // block exists (block indices clamp to the last block; K rows stored
    // after the last block are never read), and inactive waves (head
    // groups past the query's) run q.k on zero queries, so the region up
    // to the first barrier is one straight-line block and the group
    // barriers at its end can interleave the K-row loads with the q.k
    // MFMAs. p.v stays behind `active`: the accumulators of a wave that
    // skips it are never written.
    auto step = [&](uint32_t k, attn_wide_stage<DKC, NJ> &fr, attn_wide_stage<DKC, NJ> &next) {
        const uint32_t k1 = k + 1 < nb ? k + 1 : nb - 1, k2 = k + 2 < nb ? k + 2 : nb - 1;
        if (two_stages) attn_wide_load_k<DKC, NJ>(p, kbase, slots + k2 * B, tid, fr);
        sglkv_f32x4 sc[2];
        attn_wide_qk<DKC, NJ, false>(ks, qf, kc0, g, r, lane, sc, sxw);
        attn_wide_store_v<DKC, NJ>(vs, tid, ra);
        attn_wide_load_v<DKC, NJ>(p, vbase, slots + k1 * B, tid, ra);
        // Slot reads, then row loads (K with two stages, V with one) between
        // the q.k MFMAs, LDS reads of K running QK_AHEAD k-steps ahead.
        constexpr uint32_t vmem = two_stages ? G::KPT + (G::RTHREADS ? 1 : 0) : G::VPT;
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 + 2 * G::QK_AHEAD, 0);
#pragma unroll
        for (uint32_t c = 0; c < G::KH; ++c) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
            if (c < vmem) __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
            if (c + G::QK_AHEAD < G::KH) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        }
        __syncthreads();
        if (two_stages) {
            attn_wide_store_k<DKC, NJ>(ks, tid, next);
        } else {  // the one stage: block k+1's rows to LDS, then block k+2's loads
            attn_wide_store_k<DKC, NJ>(ks, tid, ra);
            attn_wide_load_k<DKC, NJ>(p, kbase, slots + k2 * B, tid, ra);
        }
        if (active) attn_wide_pv<false, DKC, NJ, false>(p, vs, sc, sxo, slots + k * B, j0, g, r, lane, st, &over);
        __syncthreads();
    };
    for (uint32_t k = 0; k < nb; k += 2) {
        step(k, ra, rb);
        if (k + 1 >= nb) break;
        step(k + 1, rb, ra);
    }
    if (active && __any(over) && lane == 0) *redo = 1;
    __syncthreads();
    // Read as a wave-uniform value, so the branch is a scalar one.
    if (__builtin_amdgcn_readfirstlane(*redo)) {
        // A block outran the fixed reference by more than the bound: the
        // split again, one block at a time, with the running maximum. The
        // queries are read again rather than kept from the main loop, whose
        // registers are then free for this path's exact p.v.
        attn_state_init(st);
        sglkv_u16x8 qr[G::KH];
        load_queries(qr);
        for (uint32_t k = 0; k < nb; ++k) {
            attn_wide_load_k<DKC, NJ>(p, kbase, slots + k * B, tid, ra);
            attn_wide_load_v<DKC, NJ>(p, vbase, slots + k * B, tid, ra);
            attn_wide_store_k<DKC, NJ>(ks, tid, ra);
            attn_wide_store_v<DKC, NJ>(vs, tid, ra);
            __syncthreads();
            sglkv_f32x4 sc[2];
            if (active) attn_wide_qk<DKC, NJ>(ks, qr, kc0, g, r, lane, sc, sxw);
            __syncthreads();
            if (active) attn_wide_pv<true, DKC, NJ>(p, vs, sc, sxo, slots + k * B, j0, g, r, lane, st, &over);
            __syncthreads();
        }
    } else if (st.m_run == -INFINITY) {
        st.m_run = -3.402823466e+38f;  // no valid token: the record's m as the exact path leaves it
    }
    if (active) attn_finish<G::NJH>(p, w, g, r, st);
}

// ---- Latent body: MLA decode, 32 query heads per wave ----
//
// For MLA's shape (K rows of 576 dims, V rows of 512, 128 query heads over
// one KV head) the wide body's two waves per 16-head group read every staged
// K and V byte once per 16 heads, and its staging registers leave room for
// little LDS read-ahead. Here a workgroup of four waves (one per SIMD) owns
// (query, KV head, up to 128 query heads, split) and wave w serves heads
// 32w .. 32w+31 with v_mfma_f32_32x32x16_bf16, so LDS is read once per 32
// heads:
//  - q.k: S[token][head] = K (A operand: lane l holds token l%32, dims
//    8(l/32) .. +7 of each 16-dim step, read from LDS) x Q^T (B operand: the
//    lane's head, 36 steps of 8 dims held in 144 VGPRs). S comes out with
//    lane l holding head l%32 and tokens 8(r/4) + 4(l/32) + r%4, r < 16.
//  - p.v: O[head][dim] += P (A operand) x V (B operand). P's k index
//    8(l/32) + i of step s is token 16s + 4(l/32) + i (i < 4) or
//    16s + 8 + 4(l/32) + i - 4, exactly the tokens S left in the lane, so P
//    needs no lane movement. V's B operand comes from two transposing LDS
//    reads (ds_read_b64_tr_b16) per tile, lane (16c + L) of each half-wave
//    addressing token 4(l/32) + L/4 (+8), dims 16c + 4(L%4) of the 32-dim
//    tile. O is 16 tiles of 16 floats: 256 accumulator registers.
//  - K and V rows go from HBM straight into LDS (global_load_lds_dwordx4:
//    lane i's 16 bytes land at M0 + 16 i), so no staging register holds
//    them. A K row's dims [0, 512) are one such load into a row of 1,040
//    bytes (rows 4 banks apart: the q.k reads of 16 tokens hit 64 distinct
//    banks); dims [512, 576) of 8 rows are one load into rows of 128 bytes,
//    piece i of row t stored at (i ^ (t/2 % 8)) so that the q.k reads are
//    conflict-free there too. A V row is one load into a row of 1,088
//    bytes (16 banks apart: the transposing reads of a half-wave cover 64
//    distinct banks). Each wave loads 8 of a block's 32 rows.
//  - Pipeline: two K stages and two V stages. Iteration k waits for K(k)
//    (barrier A), issues V(k+1) into the other V stage, runs q.k, waits for
//    V(k) (barrier B), issues K(k+2) into the K stage q.k has just read, and
//    runs softmax and p.v. The barriers wait for the wave's older loads only
//    (s_waitcnt vmcnt(17): the newest K and V issues stay in flight), so up
//    to three blocks' rows are in flight; every issue is the same 9 (K) or
//    8 (V) loads, blocks past the chunk reading the zero row, so the counts
//    hold.
//  - Softmax with the wide body's fixed reference: the first valid block
//    fixes each head's reference maximum and p = 2^(x - m) after it, so the
//    loop never touches O outside the MFMAs. If a block outruns the
//    reference by more than SGLKV_ATTN_FIXED_MAX_LOG2, the workgroup runs
//    the split again twice: once for each head's true maximum (q.k only),
//    then in full with that maximum as the reference.

typedef float sglkv_f32x16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kLatB = SGLKV_ATTN_TOKENS;
constexpr uint32_t kLatThreads = 64 * SGLKV_ATTN_LATENT_WAVES;
constexpr uint32_t kLatKSteps = 36;                             // 16-dim q.k steps over 576 dims
constexpr uint32_t kLatNT = 16;                                 // 32-dim p.v tiles over 512 dims
constexpr uint32_t kLatKP = 1040, kLatTP = 128, kLatVP = 1088;  // LDS row pitches (bytes)
constexpr uint32_t kLatKMain = kLatB * kLatKP;
constexpr uint32_t kLatK = SGLKV_ATTN_LATENT_KSTAGE, kLatV = SGLKV_ATTN_LATENT_VSTAGE;
constexpr uint32_t kLatLoadsK = 9, kLatLoadsV = 8;  // loads one wave issues per block
constexpr uint32_t kLatAhead = 4;                   // MFMA steps the LDS reads run ahead
static_assert(kLatKMain + kLatB * kLatTP == kLatK && kLatB * kLatVP == kLatV, "stage layout");
static_assert(kLatB == 8 * SGLKV_ATTN_LATENT_WAVES && SGLKV_ATTN_LATENT_HEADS == 32 * SGLKV_ATTN_LATENT_WAVES,
              "8 rows and 32 heads per wave");
static_assert(SGLKV_ATTN_LATENT_LDS_BYTES == 2 * (kLatK + kLatV) + 4 * SGLKV_ATTN_WIDE_SLOTS + 16,
              "the host sizes the same LDS");

__device__ __forceinline__ sglkv_f32x16 attn_mfma32(sglkv_u16x8 a, sglkv_u16x8 b, sglkv_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(attn_as_bf16(a), attn_as_bf16(b), c, 0, 0, 0);
}

// Row loads into LDS: global_load_lds_dwordx4 takes the LDS address from
// M0 and puts lane i's 16 bytes at M0 + 16 i. They are written out rather
// than through the compiler's builtin, which makes every later LDS read that
// it cannot prove disjoint wait for all such loads in flight (vmcnt(0)); the
// barriers of the latent body do the waiting instead. Each row is read once
// per workgroup, so the loads are non-temporal (nt): measured on the MLA
// decode, 132 -> 114 us per launch.
__device__ __forceinline__ uint32_t attn_lat_lds_at(const uint8_t *dst) {
    // dst is uniform (wave-indexed); readfirstlane tells the compiler so.
    return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t *)dst)));
}

// 16 bytes at src (per lane) into LDS at dst + 16 * lane.
__device__ __forceinline__ void attn_lat_load(uint64_t src, const uint8_t *dst) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt\n\ts_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(src), "s"(attn_lat_lds_at(dst)));
}

// ok ? a : z per lane, as two v_cndmask_b32 (see attn_sel64x2).
__device__ __forceinline__ uint64_t attn_sel64(bool ok, uint64_t a, uint64_t z) {
    const uint32_t m = ok ? 1u : 0u;
    uint32_t xl, xh;
    asm("v_cmp_ne_u32 vcc, 0, %2\n\t"
        "v_cndmask_b32 %0, %3, %4, vcc\n\t"
        "v_cndmask_b32 %1, %5, %6, vcc"
        : "=&v"(xl), "=&v"(xh)
        : "v"(m), "v"(static_cast<uint32_t>(z)), "v"(static_cast<uint32_t>(a)), "v"(static_cast<uint32_t>(z >> 32)),
          "v"(static_cast<uint32_t>(a >> 32))
        : "vcc");
    return (static_cast<uint64_t>(xh) << 32) | xl;
}

// x of lane l ^ 16 and of lane l ^ 32 (a wave of 64): gfx950's row-swap
// permutes (v_permlane16_swap_b32, v_permlane32_swap_b32), with no LDS
// round trip. A swap of x with itself leaves the partner row's x in one of
// the two results, chosen by the lane's own row.
__device__ __forceinline__ float attn_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}

__device__ __forceinline__ float attn_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// x = ok ? a : z and y = ok ? b : z per lane, as v_cndmask_b32s, which the
// compiler cannot turn into a branch around the computation of a and b.
__device__ __forceinline__ void attn_sel64x2(bool ok, uint64_t a, uint64_t b, uint64_t z, uint64_t &x,
                                             uint64_t &y) {
    const uint32_t m = ok ? 1u : 0u;
    uint32_t xl, xh, yl, yh;
    asm("v_cmp_ne_u32 vcc, 0, %4\n\t"
        "v_cndmask_b32 %0, %5, %6, vcc\n\t"
        "v_cndmask_b32 %1, %7, %8, vcc\n\t"
        "v_cndmask_b32 %2, %5, %9, vcc\n\t"
        "v_cndmask_b32 %3, %7, %10, vcc"
        : "=&v"(xl), "=&v"(xh), "=&v"(yl), "=&v"(yh)
        : "v"(m), "v"(static_cast<uint32_t>(z)), "v"(static_cast<uint32_t>(a)), "v"(static_cast<uint32_t>(z >> 32)),
          "v"(static_cast<uint32_t>(a >> 32)), "v"(static_cast<uint32_t>(b)), "v"(static_cast<uint32_t>(b >> 32))
        : "vcc");
    x = (static_cast<uint64_t>(xh) << 32) | xl;
    y = (static_cast<uint64_t>(yh) << 32) | yl;
}

// Four loads: lane l's 16 bytes of load i from a[i] to LDS at
// at + i * PITCH + 16 l (non-temporal).
template <uint32_t PITCH>
__device__ __forceinline__ void attn_lat_load4v(const uint64_t *a, uint32_t at) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off nt\n\t"
        "s_add_u32 m0, %1, %6\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %3, off nt\n\t"
        "s_add_u32 m0, %1, %7\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %4, off nt\n\t"
        "s_add_u32 m0, %1, %8\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %5, off nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "s"(at), "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "n"(PITCH), "n"(2 * PITCH), "n"(3 * PITCH)
        : "scc");
}

// Eight rows: row i's 1 KiB from a[i] (the same in every lane; lane l's 16
// bytes at a[i] + 16 l) into LDS at at + i * PITCH. The leading s_nop 4
// covers a VALU (readlane) write of a[i] just before; each M0 write is one
// wait state ahead of the load that reads it.
template <uint32_t PITCH>
__device__ __forceinline__ void attn_lat_load8(const uint64_t (&a)[8], uint32_t at) {
    uint32_t save;
    asm volatile(
        "s_nop 4\n\ts_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %3 nt\n\t"
        "s_add_u32 m0, %2, %11\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %4 nt\n\t"
        "s_add_u32 m0, %2, %12\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %5 nt\n\t"
        "s_add_u32 m0, %2, %13\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %6 nt\n\t"
        "s_add_u32 m0, %2, %14\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %7 nt\n\t"
        "s_add_u32 m0, %2, %15\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %8 nt\n\t"
        "s_add_u32 m0, %2, %16\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %9 nt\n\t"
        "s_add_u32 m0, %2, %17\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %10 nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(16 * (threadIdx.x & 63)), "s"(at), "s"(a[0]), "s"(a[1]), "s"(a[2]), "s"(a[3]), "s"(a[4]), "s"(a[5]),
          "s"(a[6]), "s"(a[7]), "n"(PITCH), "n"(2 * PITCH), "n"(3 * PITCH), "n"(4 * PITCH), "n"(5 * PITCH),
          "n"(6 * PITCH), "n"(7 * PITCH)
        : "scc");
}

__device__ __forceinline__ uint64_t attn_lat_row(const sglkv_attn_params &p, uint64_t base, uint32_t s,
                                                 uint32_t stride) {
    return base + static_cast<uint64_t>(s >> p.page_shift) * p.page_stride32 +
           static_cast<uint64_t>(s & ((1u << p.page_shift) - 1)) * stride;
}

// Row address of the token whose slot is s (the zero row for an invalid
// slot or a block past the chunk).
__device__ __forceinline__ uint64_t attn_lat_row_or_zero(const sglkv_attn_params &p, uint64_t base, uint32_t s,
                                                         uint32_t stride, bool live) {
    return live && s != kAttnInvalidSlot ? attn_lat_row(p, base, s, stride) : reinterpret_cast<uint64_t>(p.zero_row);
}

// Lane i's 64-bit value for i < 8, in SGPRs. (readlane returns int: each
// half goes through uint32_t so that the low half is not sign-extended.)
__device__ __forceinline__ void attn_lat_lanes8(uint64_t v, uint64_t (&a)[8]) {
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), i));
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), i));
        a[i] = static_cast<uint64_t>(lo) | static_cast<uint64_t>(hi) << 32;
    }
}

// Waits until at most N of this wave's vector-memory loads are in flight
// and its LDS reads are done, then joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void attn_lat_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Wave w's 9 loads of a block's K rows (slots sl; live false: a block past
// the chunk, every lane reads the zero row): rows 8w + i, dims [0, 512) at
// kst + row * 1040 (the host requires dk > 512, so every lane is inside the
// row), and the tail dims of rows 8w .. 8w+7 at kst + 32 * 1040 + 1024 w
// (lane i: row 8w + i/8, piece (i%8) ^ (row/2 % 8)), zeros at or past dk.
// Lanes 0..7 work out the eight row addresses at once.
__device__ __forceinline__ void attn_lat_issue_k(const sglkv_attn_params &p, uint64_t kbase, const uint32_t *sl,
                                                 bool live, uint32_t w, uint32_t lane, uint8_t *kst) {
    uint64_t a[8];
    attn_lat_lanes8(attn_lat_row_or_zero(p, kbase, sl[8 * w + (lane & 7)], p.key_token_stride32, live), a);
    attn_lat_load8<kLatKP>(a, attn_lat_lds_at(kst + 8 * w * kLatKP));
    const uint32_t t = 8 * w + (lane >> 3), piece = (lane & 7) ^ ((t >> 1) & 7);
    const uint32_t st = sl[t];
    const bool ok = live && st != kAttnInvalidSlot && 512 + 8 * piece < p.dk;
    const uint64_t src = ok ? attn_lat_row(p, kbase, st, p.key_token_stride32) + 1024 + 16 * piece
                            : reinterpret_cast<uint64_t>(p.zero_row) + 16 * (lane & 7);
    attn_lat_load(src, kst + kLatKMain + 1024 * w);
}

// Wave w's 8 loads of a block's V rows: row 8w + i at vst + row * 1088
// (the host requires dv = 512: every lane is inside the row).
__device__ __forceinline__ void attn_lat_issue_v(const sglkv_attn_params &p, uint64_t vbase, const uint32_t *sl,
                                                 bool live, uint32_t w, uint32_t lane, uint8_t *vst) {
    uint64_t a[8];
    attn_lat_lanes8(attn_lat_row_or_zero(p, vbase, sl[8 * w + (lane & 7)], p.value_token_stride32, live), a);
    attn_lat_load8<kLatVP>(a, attn_lat_lds_at(vst + 8 * w * kLatVP));
}

// q.k MFMAs with the scores in VGPRs. The compiler gives every MFMA it
// emits an accumulator in the same register file, and the 256 AGPRs are
// exactly o's, so these are written out: c = a x b (+ c). The compiler's
// hazard checks do not look inside them: the chain's first starts with 3
// wait states (a VALU write of a or b just before needs 2; between the
// chain's MFMAs there are only LDS reads), and its last adds 20 (an 8-pass
// 32x32 MFMA needs 18 before another instruction reads c). The chain reads
// its own previous result as the accumulator, which the hardware forwards.
__device__ __forceinline__ void attn_lat_mfma_first(sglkv_f32x16 &c, sglkv_u16x8 a, sglkv_u16x8 b) {
    asm("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void attn_lat_mfma_next(sglkv_f32x16 &c, sglkv_u16x8 a, sglkv_u16x8 b) {
    asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void attn_lat_mfma_last(sglkv_f32x16 &c, sglkv_u16x8 a, sglkv_u16x8 b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 3"
                 : "+v"(c)
                 : "v"(a), "v"(b));
}

// q.k of the staged block: lane l gets head l%32's scores of tokens
// 8(r/4) + 4(l/32) + r%4 in s[r].
__device__ __forceinline__ sglkv_f32x16 attn_lat_qk(const uint8_t *kst, const sglkv_u16x8 (&qf)[kLatKSteps],
                                                    uint32_t lane) {
    const uint32_t t = lane & 31, h = lane >> 5, sw = (t >> 1) & 7;
    const uint8_t *ka = kst + t * kLatKP + 16 * h;
    const uint8_t *ta = kst + kLatKMain + t * kLatTP;
    auto kread = [&](uint32_t c) {
        return *reinterpret_cast<const sglkv_u16x8 *>(c < 32 ? ka + 32 * c : ta + 16 * ((2 * (c - 32) + h) ^ sw));
    };
    // The reads run kLatAhead steps ahead of the MFMAs that use them.
    sglkv_u16x8 kf[kLatAhead];
#pragma unroll
    for (uint32_t c = 0; c < kLatAhead; ++c) kf[c] = kread(c);
    sglkv_f32x16 s;
#pragma unroll
    for (uint32_t c = 0; c < kLatKSteps; ++c) {
        // sched_barrier(0): the scheduler keeps this order (it would sink
        // each read next to its MFMA otherwise).
        __builtin_amdgcn_sched_barrier(0);
        const sglkv_u16x8 a = kf[c % kLatAhead];
        if (c + kLatAhead < kLatKSteps) kf[c % kLatAhead] = kread(c + kLatAhead);
        if (c == 0)
            attn_lat_mfma_first(s, a, qf[c]);
        else if (c + 1 < kLatKSteps)
            attn_lat_mfma_next(s, a, qf[c]);
        else
            attn_lat_mfma_last(s, a, qf[c]);
    }
    __builtin_amdgcn_sched_barrier(0);
    return s;
}

__device__ __forceinline__ attn_i16x4 attn_lat_vtr(const uint8_t *at) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) attn_i16x4 *)(reinterpret_cast<uintptr_t>(at)));
}

// o += P x V over the staged block (pa: the probabilities, bf16, as the A
// operand of the two 16-token steps; EXACT: pa[2 + i] holds the lo halves,
// each step taken twice, hi then lo). MFMA j is tile j/2, step j%2; its B
// operand's two transposing reads run kLatAhead MFMAs ahead.
template <bool EXACT>
__device__ __forceinline__ void attn_lat_pv(const uint8_t *vst, const sglkv_u16x8 (&pa)[EXACT ? 4 : 2],
                                            sglkv_f32x16 (&o)[kLatNT], uint32_t lane) {
    const uint32_t L = lane & 15, c = (lane >> 4) & 1, h = lane >> 5;
    const uint8_t *va = vst + (4 * h + (L >> 2)) * kLatVP + 32 * c + 8 * (L & 3);
    auto vread = [&](uint32_t j) {
        const uint8_t *at = va + 16 * (j & 1) * kLatVP + 64 * (j >> 1);
        const attn_i16x4 lo = attn_lat_vtr(at), hi = attn_lat_vtr(at + 8 * kLatVP);
        return sglkv_u16x8{(uint16_t)lo[0], (uint16_t)lo[1], (uint16_t)lo[2], (uint16_t)lo[3],
                           (uint16_t)hi[0], (uint16_t)hi[1], (uint16_t)hi[2], (uint16_t)hi[3]};
    };
    sglkv_u16x8 vf[kLatAhead];
#pragma unroll
    for (uint32_t j = 0; j < kLatAhead; ++j) vf[j] = vread(j);
#pragma unroll
    for (uint32_t j = 0; j < 2 * kLatNT; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        const sglkv_u16x8 b = vf[j % kLatAhead];
        if (j + kLatAhead < 2 * kLatNT) vf[j % kLatAhead] = vread(j + kLatAhead);
        o[j >> 1] = attn_mfma32(pa[j & 1], b, o[j >> 1]);
        if (EXACT) o[j >> 1] = attn_mfma32(pa[2 + (j & 1)], b, o[j >> 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Scores of the lane's 16 tokens in log2 units (-inf where the token is
// invalid: bit t of vm clear) and their maximum over the head's 32 tokens.
__device__ __forceinline__ float attn_lat_scores(const sglkv_attn_params &p, const sglkv_f32x16 &s, uint64_t vm,
                                                 uint32_t lane, float (&x)[16]) {
    const uint32_t h = lane >> 5;
    float mx = -INFINITY;
    if (static_cast<uint32_t>(vm) == 0xFFFFFFFFu) {  // every token valid (the same in every lane)
#pragma unroll
        for (uint32_t r = 0; r < 16; ++r) {
            x[r] = s[r] * p.scale_log2;
            mx = fmaxf(mx, x[r]);
        }
    } else {
#pragma unroll
        for (uint32_t r = 0; r < 16; ++r) {
            const uint32_t tok = 8 * (r >> 2) + 4 * h + (r & 3);
            x[r] = ((vm >> tok) & 1) ? s[r] * p.scale_log2 : -INFINITY;
            mx = fmaxf(mx, x[r]);
        }
    }
    return fmaxf(mx, __shfl_xor(mx, 32));
}

// Validity of the block's 32 tokens (bit t), from its slots.
__device__ __forceinline__ uint64_t attn_lat_valid(const uint32_t *sl, uint32_t lane) {
    return __ballot(sl[lane & 31] != kAttnInvalidSlot);
}

// Softmax of one block against the fixed reference m_run (set by the first
// valid block), l_part += the lane's p, pa = p in bf16 (EXACT: hi in pa[0..1],
// lo in pa[2..3]); *over when the block's maximum passes the reference by
// more than the bound.
template <bool EXACT>
__device__ __forceinline__ void attn_lat_softmax(const sglkv_attn_params &p, const sglkv_f32x16 &s, uint64_t vm,
                                                 uint32_t lane, float &m_run, float &l_part,
                                                 sglkv_u16x8 (&pa)[EXACT ? 4 : 2], bool &over) {
    float x[16];
    const float mx = attn_lat_scores(p, s, vm, lane, x);
    if (m_run == -INFINITY) m_run = mx;
    const float m_ref = m_run == -INFINITY ? 0.0f : m_run;
    over = over || mx > m_ref + SGLKV_ATTN_FIXED_MAX_LOG2;
    float psum = 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < 16; ++r) {
        // v_exp_f32: 2^y, 0 below the normal range (x = -inf for an invalid
        // token gives exactly 0).
        const float pr = __builtin_amdgcn_exp2f(fminf(x[r] - m_ref, SGLKV_ATTN_FIXED_MAX_LOG2));
        psum += pr;
        if (EXACT)
            attn_split_bf16(pr, pa[r >> 3], pa[2 + (r >> 3)], r & 7);
        else
            pa[r >> 3][r & 7] = attn_to_bf16(pr);
    }
    l_part += psum;
}

template <bool EXACT>
__device__ __forceinline__ void attn_latent_body(const sglkv_attn_params &p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t attn_lat_lds[];
    uint8_t *const k0 = attn_lat_lds, *const k1 = attn_lat_lds + kLatK;
    uint8_t *const v0 = attn_lat_lds + 2 * kLatK, *const v1 = v0 + kLatV;
    uint32_t *slots = reinterpret_cast<uint32_t *>(attn_lat_lds + 2 * (kLatK + kLatV));
    uint32_t *redo = slots + SGLKV_ATTN_WIDE_SLOTS;
    // w through readfirstlane: the compiler then keeps what derives from it
    // (head range, LDS row addresses) in SGPRs rather than in every lane.
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);

    // Workgroup -> (query, KV head, block of 128 query heads), split.
    const uint32_t hblocks = (p.group + SGLKV_ATTN_LATENT_HEADS - 1) / SGLKV_ATTN_LATENT_HEADS;
    uint64_t bx = blockIdx.x;
    const uint64_t q = bx % p.query_count;
    bx /= p.query_count;
    const uint32_t kvh = static_cast<uint32_t>(bx % p.kv_heads);
    const uint32_t hb = static_cast<uint32_t>(bx / p.kv_heads);
    const uint32_t split = blockIdx.y;
    uint64_t start = 0, len = 0;
    if (!attn_metadata(p, q, tid == 0 && split == 0 && hb == 0 && kvh == 0, &start, &len)) return;
    const uint64_t t0 = static_cast<uint64_t>(split) * p.chunk_tokens;
    if (t0 >= len || hb >= hblocks) return;
    const uint64_t t1 = len < t0 + p.chunk_tokens ? len : t0 + p.chunk_tokens;
    const uint32_t nb = static_cast<uint32_t>((t1 - t0 + kLatB - 1) / kLatB);  // <= SLOTS / B (host bound)
    const uint32_t hw = hb * SGLKV_ATTN_LATENT_HEADS + 32 * w;  // the wave's first head in the KV group
    const uint32_t nh = hw >= p.group ? 0 : (p.group - hw < 32 ? p.group - hw : 32);
    const bool active = nh > 0;
    const uint64_t h0 = static_cast<uint64_t>(kvh) * p.group + hw;

    if (tid == 0) *redo = 0;
    for (uint32_t i = tid; i < nb * kLatB; i += kLatThreads) {
        const uint64_t tok = t0 + i;
        slots[i] = attn_wide_slot(p, tok < t1 ? p.sequence_slots[start + tok] : 0, tok, t1);
    }
    __syncthreads();

    const uint64_t pool = reinterpret_cast<uint64_t>(p.pool);
    const uint64_t kbase = pool + p.key_offset + kvh * p.key_head_stride;
    const uint64_t vbase = pool + p.value_offset + kvh * p.value_head_stride;
    auto blk = [&](uint32_t b) { return slots + (b < nb ? b : nb - 1) * kLatB; };

    sglkv_f32x16 o[kLatNT];
#pragma unroll
    for (uint32_t n = 0; n < kLatNT; ++n) o[n] = sglkv_f32x16{};
    float m_run = -INFINITY, l_part = 0.0f;
    bool over = false;

    attn_lat_issue_k(p, kbase, blk(0), true, w, lane, k0);
    attn_lat_issue_v(p, vbase, blk(0), true, w, lane, v0);
    attn_lat_issue_k(p, kbase, blk(1), 1 < nb, w, lane, k1);
    // Queries, loaded while the first rows land: lane l holds head l%32,
    // dims 16c + 8(l/32) .. +7 of step c.
    sglkv_u16x8 qf[kLatKSteps];
#pragma unroll
    for (uint32_t c = 0; c < kLatKSteps; ++c) {
        const uint32_t d = 16 * c + 8 * (lane >> 5);
        qf[c] = sglkv_u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        if ((lane & 31) < nh && d < p.dk)
            qf[c] = *reinterpret_cast<const sglkv_u16x8 *>(p.queries + (q * p.query_heads + h0 + (lane & 31)) * p.dk + d);
    }
    // Every load so far (the first rows, which the compiler does not track,
    // and the queries, which it does) is complete before the loop, whose
    // waits then count the row loads alone (s_waitcnt vmcnt(0), lgkmcnt and
    // expcnt left at their maxima).
    __builtin_amdgcn_s_waitcnt(0x0F70);
    // Iteration k with stages (kc, vc) holding block k; (vn) takes block
    // k+1's V rows, kc block k+2's K rows.
    // Iteration k: stages kc and vc hold block k; vn takes block k+1's V
    // rows, kc (once q.k has read it) block k+2's K rows. A wave without
    // heads runs the loop on zero queries and writes nothing, so the loop
    // has no branch around the accumulators.
    for (uint32_t k = 0; k < nb; ++k) {
        uint8_t *const kc = (k & 1) ? k1 : k0;
        uint8_t *const vc = (k & 1) ? v1 : v0;
        uint8_t *const vn = (k & 1) ? v0 : v1;
        attn_lat_barrier<kLatLoadsK + kLatLoadsV>();  // K(k) in LDS; p.v(k-1) done
        attn_lat_issue_v(p, vbase, blk(k + 1), k + 1 < nb, w, lane, vn);
        const sglkv_f32x16 s = attn_lat_qk(kc, qf, lane);
        attn_lat_barrier<kLatLoadsV + kLatLoadsK>();  // V(k) in LDS; q.k(k) done
        attn_lat_issue_k(p, kbase, blk(k + 2), k + 2 < nb, w, lane, kc);
        sglkv_u16x8 pa[EXACT ? 4 : 2];
        attn_lat_softmax<EXACT>(p, s, attn_lat_valid(blk(k), lane), lane, m_run, l_part, pa, over);
        attn_lat_pv<EXACT>(vc, pa, o, lane);
    }
    // Every row load (the zero rows issued past the chunk too) has landed:
    // __syncthreads would not wait for them (its fence orders LDS and
    // stores, and the compiler does not see these loads).
    attn_lat_barrier<0>();
    if (active && __any(over) && lane == 0) *redo = 1;
    __syncthreads();
    // Read as a wave-uniform value, so the branch is a scalar one.
    if (__builtin_amdgcn_readfirstlane(*redo)) {
        // A block outran the fixed reference: each head's true maximum over
        // the split (q.k only), then the split again with that maximum as
        // the reference, which no block can outrun.
        float m_true = -INFINITY;
        for (uint32_t k = 0; k < nb; ++k) {
            attn_lat_issue_k(p, kbase, blk(k), true, w, lane, k0);
            attn_lat_barrier<0>();
            float x[16];
            m_true = fmaxf(m_true,
                           attn_lat_scores(p, attn_lat_qk(k0, qf, lane), attn_lat_valid(blk(k), lane), lane, x));
            __syncthreads();
        }
#pragma unroll
        for (uint32_t n = 0; n < kLatNT; ++n) o[n] = sglkv_f32x16{};
        m_run = m_true;
        l_part = 0.0f;
        for (uint32_t k = 0; k < nb; ++k) {
            attn_lat_issue_k(p, kbase, blk(k), true, w, lane, k0);
            attn_lat_issue_v(p, vbase, blk(k), true, w, lane, v0);
            attn_lat_barrier<0>();
            sglkv_u16x8 pa[EXACT ? 4 : 2];
            attn_lat_softmax<EXACT>(p, attn_lat_qk(k0, qf, lane), attn_lat_valid(blk(k), lane), lane, m_run, l_part, pa,
                             over);
            attn_lat_pv<EXACT>(v0, pa, o, lane);
            __syncthreads();
        }
    }
    if (!active) return;
    if (m_run == -INFINITY) m_run = -3.402823466e+38f;  // no valid token: the record's m as the other bodies leave it

    // Output (one split) or the split's scaled fp16 record: o[n][r] is head
    // 8(r/4) + 4(l/32) + r%4, dim 32n + l%32; m and l of head l%32. dv is
    // 512 (the host takes this body only then).
    const float l_tot = l_part + __shfl_xor(l_part, 32);
    // The lane index as a fresh value: derived from the prologue's, it (and
    // the head-row index computed from it there) would be kept live across
    // the loop, where every register is taken, and so spilled.
    uint32_t lane_e = lane;
    asm volatile("" : "+v"(lane_e));
    const uint32_t hl = lane_e & 31, hh = lane_e >> 5;
    if (p.splits == 1) {
        float linv[16];
#pragma unroll
        for (uint32_t r = 0; r < 16; ++r) linv[r] = 1.0f / __shfl(l_tot, 8 * (r >> 2) + 4 * hh + (r & 3));
        uint16_t *out = p.output + (q * p.query_heads + h0 + 4 * hh) * 512 + hl;
        // Each accumulator is read out (v_accvgpr_read) right where it is
        // scaled and stored. Left to the compiler, all 256 are copied to
        // VGPRs at the loop's end, which do not hold them. The last MFMA
        // writing them is at least 20 wait states back (the nops; an 8-pass
        // 32x32 MFMA needs 18 before its result is read).
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3");
#pragma unroll
        for (uint32_t n = 0; n < kLatNT; ++n) {
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) {
                if (8 * (r >> 2) + 4 * hh + (r & 3) >= nh) continue;
                float x;
                asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(o[n][r]));
                out[(8 * (r >> 2) + (r & 3)) * 512 + 32 * n] = attn_to_bf16(x * linv[r]);
            }
        }
    } else {
        // Scaled fp16 record: a = max |o| over the head's 512 dims (the
        // lane's 16 values, then the 32 lanes of its half-wave), y = o / a.
        // y's rounding moves o by at most 2^-11 |o| + 2^-25 a.
        // Head h's a reaches lane h of the first half-wave, which holds h's
        // m and l, through 128 bytes of LDS per wave (the K stage, unused
        // after the loop); each head's (m, l, a, 0) goes out as one 16-byte
        // store.
        float *const a_lds = reinterpret_cast<float *>(k0) + 32 * w;
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3");
#pragma unroll
        for (uint32_t r = 0; r < 16; ++r) {
            const uint32_t head = 8 * (r >> 2) + 4 * hh + (r & 3);
            float a = 0.0f;
#pragma unroll
            for (uint32_t n = 0; n < kLatNT; ++n) {
                float x;
                asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(o[n][r]));
                a = fmaxf(a, fabsf(x));
            }
#pragma unroll
            for (uint32_t d = 1; d < 32; d <<= 1) a = fmaxf(a, __shfl_xor(a, d));
            if (hl == 0) a_lds[head] = a;
            if (head >= nh) continue;
            const uint64_t rec = (q * p.query_heads + h0 + head) * p.splits + split;
            const float inv = a > 0.0f ? 1.0f / a : 0.0f;
            uint16_t *py = attn_rec_y(p, rec) + hl;
#pragma unroll
            for (uint32_t n = 0; n < kLatNT; ++n) {
                float x;
                asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(o[n][r]));
                __builtin_nontemporal_store(__builtin_bit_cast(uint16_t, static_cast<_Float16>(x * inv)),
                                            py + 32 * n);
            }
        }
        if (hh == 0 && hl < nh) {
            const sglkv_f32x4 mla = {m_run, l_tot, a_lds[hl], 0.0f};
            __builtin_nontemporal_store(mla, reinterpret_cast<sglkv_f32x4 *>(attn_rec_mla(p, q, split, h0 + hl)));
        }
    }
}

// ---- Staged bodies: GQA decode with K and V head dims D = 128 or 64 ----
//
// The pipelined body's loads put each 16-byte piece of a row into a
// register, and its V transpose goes through LDS store by store. Here one
// wave (a workgroup) owns (query, KV head, up to 16 query heads, split), as
// there, but its K and V rows go from HBM straight into LDS with
// non-temporal global_load_lds_dwordx4: one load moves the 2D-byte head
// slices of 512/D tokens (4 at D = 128, 8 at D = 64), D/8 loads a 32-token
// block, with no register staging. Two stages: while block k is computed,
// block k+1 is loading. One wave needs no barrier: s_waitcnt vmcnt(D/8)
// leaves the newer block's loads in flight.
//  - q.k is the pipelined body's (K as the A operand, lane (g, r) reading
//    token 8(r/4) + 4b + r%4, dims 32c + 8g), from LDS; the queries are
//    the B operand in registers.
//  - p.v takes V through transposing reads (ds_read_b64_tr_b16): lane r of
//    16-lane group g addresses token 8g + r/4 (then 8g + 4 + r/4), dims
//    16j + 4(r%4), which yields V[8g .. 8g+7][16j + r], the order the
//    probabilities leave q.k in.
//  - Piece (16 bytes) pc of token t's K row sits at position pc ^ mask(t)
//    of its LDS row, the mask chosen so that the 16 tokens one q.k read
//    covers land in 16 distinct 16-byte bank groups: at D = 128 (256-byte
//    rows) mask = (t & 3) | 4(t >> 3); at D = 64 (128-byte rows, two per
//    bank period, t & 1 already apart) mask = (t >> 1 & 1) | 2(t >> 3).
//    V pieces: at D = 128 pc ^ (2(t & 3) | 8((t >> 3) & 1)), at D = 64
//    pc ^ (2((t >> 1) & 1) | 4((t >> 3) & 1)): the 4 tokens x 4 dims of a
//    16-lane transposing read, and the two 16-lane groups read together,
//    land in distinct banks. Each load's lane fetches the global piece its
//    LDS position holds.
//  - The slot table keeps token t of a block at entry (D/16)(t % T) + t/T
//    (T = 512/D tokens per load), so the D/16 tokens Tj + c that lanes
//    with c = lane / (D/8) load come in 16-byte reads.
//  - Online softmax with lazy rescaling (o is D/4 registers): the
//    reference maximum moves only when a block's maximum passes it by more
//    than 8 log2 units.
//  - Tokens past the sequence's end read the zero row and score -inf. A
//    slot that fails its range check (which sets the error word, so the
//    launch reports an error and its outputs carry no meaning) reads the
//    zero row too.

template <uint32_t D>
struct attn_stg {
    static constexpr uint32_t ROW = 2 * D;                   // bytes of one token's head slice
    static constexpr uint32_t PIECES = D / 8;                // 16-byte pieces per row
    static constexpr uint32_t TPL = 1024 / ROW;              // tokens per load
    static constexpr uint32_t LOADS = kLatB / TPL;           // loads per block, K (and as many V)
    static constexpr uint32_t V = kLatB * ROW;               // V rows' offset in a stage
    static constexpr uint32_t STAGE = 2 * V;                 // bytes of a stage
    static constexpr uint32_t KC = D / 32;                   // q.k steps
    static constexpr uint32_t NJ = D / 16;                   // p.v tiles
    static_assert((D == 64 || D == 128 || D == 256) &&
                      STAGE * SGLKV_ATTN_STAGED_STAGES + 4 * SGLKV_ATTN_STAGED_SLOTS ==
                          SGLKV_ATTN_STAGED_LDS_BYTES(D),
                  "stage layout");
    static_assert(2 * LOADS % 8 == 0, "whole groups of eight loads");
    // Rows of 256 and 512 bytes both start on a 256-byte bank period, so
    // dims 256 take the swizzles of dims 128 (their pieces' bit 4 is kept).
    static __device__ __forceinline__ uint32_t kpos(uint32_t t, uint32_t pc) {
        return D >= 128 ? pc ^ ((t & 3) | ((t >> 1) & 12)) : pc ^ (((t >> 1) & 1) | ((t >> 2) & 6));
    }
    static __device__ __forceinline__ uint32_t vpos(uint32_t t, uint32_t pc) {
        return D >= 128 ? pc ^ (((t & 3) << 1) | (((t >> 3) & 1) << 3))
                        : pc ^ ((((t >> 1) & 1) << 1) | (((t >> 3) & 1) << 2));
    }
    static __device__ __forceinline__ uint32_t entry(uint32_t t) { return LOADS * (t % TPL) + t / TPL; }
};

// Eight loads: lane l's 16 bytes of load i from a[i] to LDS at
// at + i * PITCH + 16 l (non-temporal).
template <uint32_t PITCH>
__device__ __forceinline__ void attn_lat_load8v(const uint64_t *a, uint32_t at) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off nt\n\t"
        "s_add_u32 m0, %1, %10\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %3, off nt\n\t"
        "s_add_u32 m0, %1, %11\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %4, off nt\n\t"
        "s_add_u32 m0, %1, %12\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %5, off nt\n\t"
        "s_add_u32 m0, %1, %13\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %6, off nt\n\t"
        "s_add_u32 m0, %1, %14\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %7, off nt\n\t"
        "s_add_u32 m0, %1, %15\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %8, off nt\n\t"
        "s_add_u32 m0, %1, %16\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %9, off nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "s"(at), "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),
          "n"(PITCH), "n"(2 * PITCH), "n"(3 * PITCH), "n"(4 * PITCH), "n"(5 * PITCH), "n"(6 * PITCH),
          "n"(7 * PITCH)
        : "scc");
}

// The lane's LOADS slot entries of a block (table entries at tb), and the
// block's 2 LOADS loads from them (live false: past the chunk, every lane
// reads the zero row) into a stage: K rows, then V rows, 1 KiB each at
// consecutive LDS offsets.
template <uint32_t D>
__device__ __forceinline__ void attn_stg_slots(const uint32_t *tb, uint32_t lane, uint32_t (&s)[attn_stg<D>::LOADS]) {
    typedef attn_stg<D> S;
    const uint32_t c = lane / S::PIECES;
#pragma unroll
    for (uint32_t h = 0; h < S::LOADS / 4; ++h) {
        const uint4 v = *reinterpret_cast<const uint4 *>(tb + S::LOADS * c + 4 * h);
        s[4 * h] = v.x;
        s[4 * h + 1] = v.y;
        s[4 * h + 2] = v.z;
        s[4 * h + 3] = v.w;
    }
}

template <uint32_t D>
__device__ __forceinline__ void attn_stg_issue(const sglkv_attn_params &p, uint64_t kbase, uint64_t vbase,
                                               const uint32_t (&s)[attn_stg<D>::LOADS], bool live, uint32_t lane,
                                               const uint8_t *stage) {
    typedef attn_stg<D> S;
    const uint32_t c = lane / S::PIECES, pc = lane % S::PIECES;
    const uint64_t zero = reinterpret_cast<uint64_t>(p.zero_row) + 16 * pc;
    const uint32_t mask = (1u << p.page_shift) - 1;
    // Each address is computed from a slot that is always in range (slot 0
    // for dead tokens) and then selected: no branches. K and V rows share
    // the token's offset (the host gives this body equal token strides, a
    // page_size and token stride below 2^24 and pages of at most 4 GiB, so
    // pos * stride fits a 24-bit multiply and 32 bits).
    // Four loads' tokens at a time (K rows, then V rows), so at most eight
    // addresses are live.
    const uint32_t at = attn_lat_lds_at(stage);
#pragma unroll
    for (uint32_t h = 0; h < S::LOADS / 4; ++h) {
        uint64_t a[8];
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t j = 4 * h + i, t = S::TPL * j + c;
            const bool ok = live && s[j] != kAttnInvalidSlot;
            const uint32_t sj = ok ? s[j] : 0u;
            const uint32_t in_page = __umul24(sj & mask, p.key_token_stride32);
            const uint64_t off = static_cast<uint64_t>(sj >> p.page_shift) * p.page_stride32 + in_page;
            attn_sel64x2(ok, kbase + off + 16 * S::kpos(t, pc), vbase + off + 16 * S::vpos(t, pc), zero, a[i],
                         a[4 + i]);
        }
        attn_lat_load4v<1024>(a, at + 4096 * h);
        attn_lat_load4v<1024>(a + 4, at + S::V + 4096 * h);
    }
}

// Softmax of one block against the running maximum (rescaling o and l),
// then o += p.v with V from the stage by transposing reads.
template <uint32_t D>
__device__ __forceinline__ void attn_stg_softmax_pv(const sglkv_attn_params &p, uint32_t g, uint32_t r,
                                                    const sglkv_f32x4 (&sc)[2], uint32_t nv,
                                                    const uint8_t *vst, attn_state_n<attn_stg<D>::NJ> &st) {
    typedef attn_stg<D> S;
    // The B operands of the p.v tiles (tile j: V[8g .. 8g+7][16j + r]) of
    // the first group of (at most eight) tiles are read first, so their
    // LDS latency passes under the softmax.
    constexpr uint32_t VG = S::NJ > 8 ? 8 : S::NJ;
    const uint32_t t0 = 8 * g + (r >> 2), t1 = t0 + 4, d4 = r & 3;
    auto vread = [&](uint32_t j) {
        const uint32_t pc = 2 * j + (d4 >> 1), half = 8 * (d4 & 1);
        const attn_i16x4 lo = attn_lat_vtr(vst + S::ROW * t0 + 16 * S::vpos(t0, pc) + half);
        const attn_i16x4 hi = attn_lat_vtr(vst + S::ROW * t1 + 16 * S::vpos(t1, pc) + half);
        return sglkv_u16x8{(uint16_t)lo[0], (uint16_t)lo[1], (uint16_t)lo[2], (uint16_t)lo[3],
                           (uint16_t)hi[0], (uint16_t)hi[1], (uint16_t)hi[2], (uint16_t)hi[3]};
    };
    sglkv_u16x8 vv[VG];
#pragma unroll
    for (uint32_t j = 0; j < VG; ++j) vv[j] = vread(j);
    // Score row 4g + e of tile b is the block's token 8g + 4b + e; the
    // first nv tokens of the block are the sequence's.
    float x[8];
#pragma unroll
    for (uint32_t b = 0; b < 2; ++b)
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) x[4 * b + e] = sc[b][e] * p.scale_log2;
    if (nv < kLatB) {
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b)
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e)
                if (8 * g + 4 * b + e >= nv) x[4 * b + e] = -INFINITY;
    }
    float mx = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    mx = fmaxf(mx, attn_xor16(mx));
    mx = fmaxf(mx, attn_xor32(mx));
    // Lazy rescaling: the reference m_run moves (and o and l are rescaled)
    // only when some head's block maximum passes it by more than 8 log2
    // units, so every weight is at most 2^8 and most blocks skip the
    // rescale. The record's (m, l, o) stay relative to the same m.
    if (__builtin_amdgcn_readfirstlane(__ballot(mx > st.m_run + 8.0f) != 0 ? 1u : 0u)) {
        const float m_new = fmaxf(st.m_run, mx);
        const float alpha = exp2f(st.m_run - m_new);
        st.l_part *= alpha;
        st.m_run = m_new;
        float arow[4];
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) arow[e] = __shfl(alpha, 4 * g + e);
#pragma unroll
        for (uint32_t j = 0; j < S::NJ; ++j)
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) st.o[j][e] *= arow[e];
    }
    sglkv_u16x8 phi, plo;
    float psum = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        const float pi = __builtin_amdgcn_exp2f(x[i] - st.m_run);  // 0 for -inf; flushes below 2^-126
        psum += pi;
        attn_split_bf16(pi, phi, plo, i);
    }
    st.l_part += psum;
#pragma unroll
    for (uint32_t j0 = 0; j0 < S::NJ; j0 += VG) {
        if (j0 > 0) {
#pragma unroll
            for (uint32_t j = 0; j < VG; ++j) vv[j] = vread(j0 + j);
        }
#pragma unroll
        for (uint32_t j = 0; j < VG; ++j) {
            st.o[j0 + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(phi), attn_as_bf16(vv[j]),
                                                                   st.o[j0 + j], 0, 0, 0);
            st.o[j0 + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(plo), attn_as_bf16(vv[j]),
                                                                   st.o[j0 + j], 0, 0, 0);
        }
    }
}

template <uint32_t D>
__device__ __forceinline__ void attn_staged_body(const sglkv_attn_params &p) {
    typedef attn_stg<D> S;
    extern __shared__ __attribute__((aligned(16))) uint8_t attn_stg_lds[];
    uint32_t *table = reinterpret_cast<uint32_t *>(attn_stg_lds + SGLKV_ATTN_STAGED_STAGES * S::STAGE);
    const uint32_t lane = threadIdx.x;
    const uint32_t g = lane >> 4, r = lane & 15;
    attn_work w;
    if (!attn_decode(p, lane, &w)) return;
    const uint32_t nb = static_cast<uint32_t>((w.t1 - w.t0 + kLatB - 1) / kLatB);  // <= SLOTS / 32 (host bound)

    // Queries (B operand of q.k): head r, dims 32c + 8g.
    sglkv_u16x8 qf[S::KC];
#pragma unroll
    for (uint32_t c = 0; c < S::KC; ++c) {
        qf[c] = sglkv_u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        if (r < w.nh)
            qf[c] = *reinterpret_cast<const sglkv_u16x8 *>(p.queries + (w.q * p.query_heads + w.h0 + r) * D +
                                                            32 * c + 8 * g);
    }
    // The chunk's slots, checked once; token t of block b at entry
    // 32 b + entry(t).
    for (uint32_t i = lane; i < nb * kLatB; i += 64) {
        const uint64_t tok = w.t0 + i;
        table[(i & ~31u) + S::entry(i & 31)] =
            attn_wide_slot(p, tok < w.t1 ? p.sequence_slots[w.start + tok] : 0, tok, w.t1);
    }
    __syncthreads();

    const uint64_t pool = reinterpret_cast<uint64_t>(p.pool);
    const uint64_t kbase = pool + p.key_offset + w.kvh * p.key_head_stride;
    const uint64_t vbase = pool + p.value_offset + w.kvh * p.value_head_stride;
    auto blk = [&](uint32_t b) { return table + (b < nb ? b : nb - 1) * kLatB; };
    auto stage = [&](uint32_t b) { return attn_stg_lds + (b % SGLKV_ATTN_STAGED_STAGES) * S::STAGE; };
    static_assert(SGLKV_ATTN_STAGED_STAGES == 2, "one block in flight ahead");
    uint32_t sl[S::LOADS];
    attn_stg_slots<D>(blk(0), lane, sl);
    attn_stg_issue<D>(p, kbase, vbase, sl, true, lane, stage(0));
    attn_stg_slots<D>(blk(1), lane, sl);
    // The query and slot loads (which the compiler tracks) are complete
    // before the loop; the loop's waits count the row loads alone.
    __builtin_amdgcn_s_waitcnt(0x0F70);

    attn_state_n<S::NJ> st;
    attn_state_init(st);
    for (uint32_t k = 0; k < nb; ++k) {
        // Block k-1's LDS reads are done before block k+1's rows overwrite
        // its stage; block k+1's slot entries were read one block ahead.
        // Then block k's loads (older than block k+1's) have landed.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        attn_stg_issue<D>(p, kbase, vbase, sl, k + 1 < nb, lane, stage(k + 1));
        attn_stg_slots<D>(blk(k + 2), lane, sl);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * S::LOADS) : "memory");
        const uint8_t *kst = stage(k);
        // The K reads of a group of q.k steps first, then the two score
        // tiles' MFMA chains interleaved (groups of 4 steps at dims 256, to
        // bound the registers the reads hold).
        constexpr uint32_t KG = S::KC > 4 ? 4 : S::KC;
        sglkv_f32x4 sc[2] = {sglkv_f32x4{0.f, 0.f, 0.f, 0.f}, sglkv_f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (uint32_t c0 = 0; c0 < S::KC; c0 += KG) {
            sglkv_u16x8 kf[2][KG];
#pragma unroll
            for (uint32_t b = 0; b < 2; ++b) {
                const uint32_t t = 8 * (r >> 2) + 4 * b + (r & 3);
#pragma unroll
                for (uint32_t c = 0; c < KG; ++c)
                    kf[b][c] = *reinterpret_cast<const sglkv_u16x8 *>(kst + S::ROW * t +
                                                                      16 * S::kpos(t, 4 * (c0 + c) + g));
            }
#pragma unroll
            for (uint32_t c = 0; c < KG; ++c)
#pragma unroll
                for (uint32_t b = 0; b < 2; ++b)
                    sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(kf[b][c]), attn_as_bf16(qf[c0 + c]),
                                                                    sc[b], 0, 0, 0);
        }
        const uint64_t left = w.t1 - w.t0 - static_cast<uint64_t>(kLatB) * k;
        attn_stg_softmax_pv<D>(p, g, r, sc, left < kLatB ? static_cast<uint32_t>(left) : kLatB, kst + S::V, st);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the zero-row loads issued past the chunk
    attn_finish(p, w, g, r, st);
}

// ---- The staged body with K in registers (dims 128, head-major pages) ----
//
// The staged layout for V (transposing reads need it in LDS), but each K
// row piece goes straight from the pool into the VGPRs of the q.k A
// operand: lane (g, r) of score tile b takes 16 bytes of token
// 8(r >> 2) + 4b + (r & 3) at dims 32c + 8g for every q.k step c. A wave's
// LDS is then its two V stages and its slot table (20 KiB at dims 128), so
// twice as many waves share a CU (eight), each with two blocks of K and up
// to two of V in flight. K loads are inline asm like the V loads (the
// compiler would count only its own loads in its waits); their registers
// pass through the wait that covers them, so no use moves above it. Steps
// c and c + 1 read the two halves of one 128-byte line. The loads carry
// sc0 nt: measured on the head-major bench (alternating runs, GB/s wall),
// 5,651 against 5,519 with the default policy, 5,601 with nt alone, 5,439
// with sc0 and 5,327 with sc1. On MI355X this body pays on head-major
// pages (a head's tokens are consecutive rows): 99.5 -> 94.3 us per launch
// on the 64-query bench; on token-major pages it took 102-114 us against
// the LDS-staged body's 95.8 whatever the policy, so those keep that one.
typedef unsigned int attn_u32x4 __attribute__((ext_vector_type(4)));

template <uint32_t D>
struct attn_kr {
    typedef attn_stg<D> S;
    static constexpr uint32_t VST = kLatB * S::ROW;  // one V stage
    static constexpr uint32_t KL = 2 * S::KC;        // K register loads per block
};

__device__ __forceinline__ attn_u32x4 attn_kr_load(uint64_t a) {
    attn_u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off sc0 nt" : "=v"(v) : "v"(a) : "memory");
    return v;
}

// K pieces of block `tb` (live false: past the chunk) into kr[b][c].
template <uint32_t D>
__device__ __forceinline__ void attn_kr_issue_k(const sglkv_attn_params &p, uint64_t kbase, const uint32_t *tb,
                                                bool live, uint32_t g, uint32_t r,
                                                attn_u32x4 (&kr)[2][attn_stg<D>::KC]) {
    typedef attn_stg<D> S;
    const uint32_t mask = (1u << p.page_shift) - 1;
    const uint64_t zero = reinterpret_cast<uint64_t>(p.zero_row);
#pragma unroll
    for (uint32_t b = 0; b < 2; ++b) {
        const uint32_t t = 8 * (r >> 2) + 4 * b + (r & 3);
        const uint32_t s = tb[S::entry(t)];
        const bool ok = live && s != kAttnInvalidSlot;
        const uint32_t sj = ok ? s : 0u;
        const uint32_t in_page = __umul24(sj & mask, p.key_token_stride32);
        const uint64_t row = attn_sel64(
            ok, kbase + static_cast<uint64_t>(sj >> p.page_shift) * p.page_stride32 + in_page, zero);
#pragma unroll
        for (uint32_t c = 0; c < S::KC; ++c) kr[b][c] = attn_kr_load(row + 16 * (4 * c + g));
    }
}

// V rows of block `tb` into a V stage (the staged layout's V half).
template <uint32_t D>
__device__ __forceinline__ void attn_kr_issue_v(const sglkv_attn_params &p, uint64_t vbase, const uint32_t *tb,
                                                bool live, uint32_t lane, const uint8_t *stage) {
    typedef attn_stg<D> S;
    uint32_t s[S::LOADS];
    attn_stg_slots<D>(tb, lane, s);
    const uint32_t c = lane / S::PIECES, pc = lane % S::PIECES;
    const uint64_t zero = reinterpret_cast<uint64_t>(p.zero_row) + 16 * pc;
    const uint32_t mask = (1u << p.page_shift) - 1;
    uint64_t a[S::LOADS];
#pragma unroll
    for (uint32_t j = 0; j < S::LOADS; ++j) {
        const uint32_t t = S::TPL * j + c;
        const bool ok = live && s[j] != kAttnInvalidSlot;
        const uint32_t sj = ok ? s[j] : 0u;
        const uint32_t in_page = __umul24(sj & mask, p.value_token_stride32);
        a[j] = attn_sel64(ok, vbase + static_cast<uint64_t>(sj >> p.page_shift) * p.page_stride32 + in_page +
                                  16 * S::vpos(t, pc),
                          zero);
    }
    const uint32_t at = attn_lat_lds_at(stage);
    if constexpr (S::LOADS == 8)
        attn_lat_load8v<1024>(a, at);
    else
        attn_lat_load4v<1024>(a, at);
}

// Waits until at most N vector-memory loads are outstanding; the K
// registers of the block pass through it.
template <uint32_t N, uint32_t KC>
__device__ __forceinline__ void attn_kr_wait(attn_u32x4 (&kr)[2][KC]) {
    if constexpr (KC == 4)
        asm volatile("s_waitcnt vmcnt(%8)"
                     : "+v"(kr[0][0]), "+v"(kr[0][1]), "+v"(kr[0][2]), "+v"(kr[0][3]), "+v"(kr[1][0]),
                       "+v"(kr[1][1]), "+v"(kr[1][2]), "+v"(kr[1][3])
                     : "n"(N)
                     : "memory");
    else
        asm volatile("s_waitcnt vmcnt(%4)"
                     : "+v"(kr[0][0]), "+v"(kr[0][1]), "+v"(kr[1][0]), "+v"(kr[1][1])
                     : "n"(N)
                     : "memory");
}

template <uint32_t D>
__device__ __forceinline__ void attn_kr_block(const sglkv_attn_params &p, uint32_t g, uint32_t r,
                                              const sglkv_u16x8 (&qf)[attn_stg<D>::KC],
                                              const attn_u32x4 (&kr)[2][attn_stg<D>::KC], const uint8_t *vst,
                                              uint32_t nv, attn_state_n<attn_stg<D>::NJ> &st) {
    typedef attn_stg<D> S;
    sglkv_f32x4 sc[2] = {sglkv_f32x4{0.f, 0.f, 0.f, 0.f}, sglkv_f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (uint32_t c = 0; c < S::KC; ++c)
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b)
            sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(__builtin_bit_cast(sglkv_u16x8, kr[b][c])),
                                                            attn_as_bf16(qf[c]), sc[b], 0, 0, 0);
    attn_stg_softmax_pv<D>(p, g, r, sc, nv, vst, st);
}

template <uint32_t D>
__device__ __forceinline__ void attn_kreg_body(const sglkv_attn_params &p) {
    typedef attn_stg<D> S;
    typedef attn_kr<D> K;
    extern __shared__ __attribute__((aligned(16))) uint8_t attn_kr_lds[];
    uint32_t *table = reinterpret_cast<uint32_t *>(attn_kr_lds + 2 * K::VST);
    const uint32_t lane = threadIdx.x;
    const uint32_t g = lane >> 4, r = lane & 15;
    attn_work w;
    if (!attn_decode(p, lane, &w)) return;
    const uint32_t nb = static_cast<uint32_t>((w.t1 - w.t0 + kLatB - 1) / kLatB);

    sglkv_u16x8 qf[S::KC];
#pragma unroll
    for (uint32_t c = 0; c < S::KC; ++c) {
        qf[c] = sglkv_u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        if (r < w.nh)
            qf[c] = *reinterpret_cast<const sglkv_u16x8 *>(p.queries + (w.q * p.query_heads + w.h0 + r) * D +
                                                            32 * c + 8 * g);
    }
    for (uint32_t i = lane; i < nb * kLatB; i += 64) {
        const uint64_t tok = w.t0 + i;
        table[(i & ~31u) + S::entry(i & 31)] =
            attn_wide_slot(p, tok < w.t1 ? p.sequence_slots[w.start + tok] : 0, tok, w.t1);
    }
    __syncthreads();

    const uint64_t pool = reinterpret_cast<uint64_t>(p.pool);
    const uint64_t kbase = pool + p.key_offset + w.kvh * p.key_head_stride;
    const uint64_t vbase = pool + p.value_offset + w.kvh * p.value_head_stride;
    auto blk = [&](uint32_t b) { return table + (b < nb ? b : nb - 1) * kLatB; };
    uint8_t *const v0 = attn_kr_lds, *const v1 = attn_kr_lds + K::VST;
    auto nvalid = [&](uint32_t k) {
        const uint64_t left = w.t1 - w.t0 - static_cast<uint64_t>(kLatB) * k;
        return left < kLatB ? static_cast<uint32_t>(left) : kLatB;
    };
    // Blocks alternate between register set A with stage v0 (even) and B
    // with v1 (odd). Loads in issue order: K(k) V(k) per block; a block's
    // wait leaves the next block's K.L + LOADS loads outstanding.
    attn_u32x4 ka[2][S::KC], kb[2][S::KC];
    attn_kr_issue_k<D>(p, kbase, blk(0), true, g, r, ka);
    attn_kr_issue_v<D>(p, vbase, blk(0), true, lane, v0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // the query and slot loads (and block 0)

    attn_state_n<S::NJ> st;
    attn_state_init(st);
    constexpr uint32_t AHEAD = K::KL + S::LOADS;
    for (uint32_t k = 0; k < nb; k += 2) {
        // p.v(k-1) read v1 before V(k+1) lands there.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        attn_kr_issue_k<D>(p, kbase, blk(k + 1), k + 1 < nb, g, r, kb);
        attn_kr_issue_v<D>(p, vbase, blk(k + 1), k + 1 < nb, lane, v1);
        attn_kr_wait<AHEAD, S::KC>(ka);
        attn_kr_block<D>(p, g, r, qf, ka, v0, nvalid(k), st);
        if (k + 1 >= nb) break;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        attn_kr_issue_k<D>(p, kbase, blk(k + 2), k + 2 < nb, g, r, ka);
        attn_kr_issue_v<D>(p, vbase, blk(k + 2), k + 2 < nb, lane, v0);
        attn_kr_wait<AHEAD, S::KC>(kb);
        attn_kr_block<D>(p, g, r, qf, kb, v1, nvalid(k + 1), st);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the loads issued past the chunk
    attn_finish(p, w, g, r, st);
}

}  // namespace

extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_v16(sglkv_attn_params p) {
    attn_body<true>(p);
}

extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void
sglkv_paged_attention_v2(sglkv_attn_params p) {
    attn_body<false>(p);
}

// Many heads per KV head: MLA widths (K <= 576, V <= 512) / dims <= 128.
extern "C" __global__ __launch_bounds__(512) void sglkv_paged_attention_wide576(sglkv_attn_params p) {
    attn_wide_body<18, 32>(p);
}

extern "C" __global__ __launch_bounds__(512) void sglkv_paged_attention_wide128(sglkv_attn_params p) {
    attn_wide_body<4, 8>(p);
}

// K and V head dims 128 / 64, up to 16 query heads per KV head, rows
// staged in LDS; for head-major pages, dims 128 also with K in registers
// and V alone in LDS. A budget of 256 registers (two waves per SIMD) makes
// the compiler keep the accumulators in VGPRs instead of copying them
// between AGPRs and VGPRs every block.
extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void
sglkv_paged_attention_staged128(sglkv_attn_params p) {
    attn_staged_body<128>(p);
}

extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void
sglkv_paged_attention_staged128k(sglkv_attn_params p) {
    attn_kreg_body<128>(p);
}

extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void
sglkv_paged_attention_staged64(sglkv_attn_params p) {
    attn_staged_body<64>(p);
}

// Dims 256 (Qwen3.5's full-attention layers): 68 KiB of LDS, two
// workgroups per CU.
extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void
sglkv_paged_attention_staged256(sglkv_attn_params p) {
    attn_staged_body<256>(p);
}

// MLA latent rows (K <= 576, V <= 512 dims), up to 128 query heads per
// workgroup.
extern "C" __global__ __launch_bounds__(256) void sglkv_paged_attention_latent(sglkv_attn_params p) {
    // Naming an accumulator register keeps the compiler's MFMA accumulators
    // in AGPRs (the 256 of o), leaving the VGPRs to the queries and scores.
    asm volatile("" ::: "a0");
    attn_latent_body<false>(p);
}

// The same with each weight fed to p.v as hi + lo bf16 values, as the other
// bodies always do (SGL_KV_ATTN_EXACT_WEIGHTS).
extern "C" __global__ __launch_bounds__(256) void sglkv_paged_attention_latent_exact(sglkv_attn_params p) {
    asm volatile("" ::: "a0");
    attn_latent_body<true>(p);
}

// Head dims exactly 128 (no per-dim masks) / up to 128.
extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_pipe128(sglkv_attn_params p) {
    attn_pipe_body<true>(p);
}

extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_pipe(sglkv_attn_params p) {
    attn_pipe_body<false>(p);
}

// Merges splits s_begin, s_begin + s_step*8 (groups of eight) of one
// (query, head)'s records into (m, l, acc) for dims d .. d+3, with a
// running maximum: each group's (m, l) pairs and o pieces load at once.
// Lanes of a group past the used splits reload the last used split and
// weigh it 0.
__device__ __forceinline__ void attn_combine_groups(const float2 *ml, const float *o, uint32_t opad, uint32_t d,
                                                    uint32_t used, uint32_t s_begin, uint32_t s_step, float &m,
                                                    float &l, float (&acc)[4]) {
    for (uint32_t s0 = s_begin; s0 < used; s0 += s_step) {
        float2 r[8];
        float4 v[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const uint32_t s = s0 + j < used ? s0 + j : used - 1;
            r[j] = ml[s];
            v[j] = *reinterpret_cast<const float4 *>(o + s * opad + d);
        }
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const bool ok = s0 + j < used;
            const float m_new = ok ? fmaxf(m, r[j].x) : m;
            const float a = exp2f(m - m_new);
            const float w = ok ? exp2f(r[j].x - m_new) : 0.0f;
            l = l * a + w * r[j].y;
            acc[0] = acc[0] * a + w * v[j].x;
            acc[1] = acc[1] * a + w * v[j].y;
            acc[2] = acc[2] * a + w * v[j].z;
            acc[3] = acc[3] * a + w * v[j].w;
            m = m_new;
        }
    }
}

// Merges the split records of one (query, head): m* = max m_s,
// out = sum_s 2^(m_s - m*) o_s / sum_s 2^(m_s - m*) l_s. Thread t handles
// dims 4t .. 4t+3 of each split's o row (one 16-byte read; rows are
// 128-byte aligned, dims past dv read the row's padding and are not
// written). A row of dv < 512 dims needs only ceil(dv / 4) threads: the
// workgroup's threads then form `sets` of that many, set i merging split
// groups i, i + sets, ..., and set 0 merges the sets' partial (m, l, o)
// through LDS, so a query split many ways waits for one memory latency per
// `sets` groups of eight splits, not per group.
extern "C" __global__ __launch_bounds__(128) void sglkv_paged_attention_combine(sglkv_attn_params p) {
    __shared__ float part[128][6];  // m, l, o[4] of each thread of sets 1..
    const uint64_t q = blockIdx.x / p.query_heads;
    const uint32_t head = static_cast<uint32_t>(blockIdx.x % p.query_heads);
    uint64_t start = 0, len = 0;
    if (!attn_metadata(p, q, false, &start, &len)) return;  // uniform over the workgroup
    const uint32_t used = static_cast<uint32_t>((len + p.chunk_tokens - 1) / p.chunk_tokens);
    const uint64_t i0 = (q * p.query_heads + head) * p.splits;
    const float2 *ml = reinterpret_cast<const float2 *>(attn_rec_ml(p, i0));
    const float *o = attn_rec_o(p, i0);
    const uint32_t opad = SGLKV_ATTN_OPAD(p.dv);
    uint16_t *out = p.output + (q * p.query_heads + head) * p.dv;
    const uint32_t pieces = (p.dv + 3) / 4;
    const uint32_t lanes = pieces < blockDim.x ? pieces : blockDim.x;
    const uint32_t sets = blockDim.x / lanes, set = threadIdx.x / lanes, tl = threadIdx.x % lanes;
    auto write = [&](uint32_t d, float m, float l, const float (&acc)[4]) {
        (void)m;
        const float linv = 1.0f / l;
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e)
            if (d + e < p.dv) out[d + e] = attn_to_bf16(acc[e] * linv);
    };
    if (sets == 1 || used <= 8) {  // (uniform over the workgroup: one query's splits)
        for (uint32_t d = 4 * threadIdx.x; d < p.dv; d += 4 * blockDim.x) {
            float m = -3.402823466e+38f, l = 0.0f, acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            attn_combine_groups(ml, o, opad, d, used, 0, 8, m, l, acc);
            write(d, m, l, acc);
        }
        return;
    }
    // One 4-dim piece per thread (4 * lanes >= dv); threads past the last
    // whole set (blockDim.x % lanes of them) only join the barrier. A set
    // with no group keeps m = -FLT_MAX, l = 0, o = 0, which the merge
    // weighs 0.
    const uint32_t d = 4 * tl;
    float m = -3.402823466e+38f, l = 0.0f, acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (set < sets) attn_combine_groups(ml, o, opad, d, used, 8 * set, 8 * sets, m, l, acc);
    if (set > 0 && set < sets) {
        float *pw = part[threadIdx.x];
        pw[0] = m;
        pw[1] = l;
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) pw[2 + e] = acc[e];
    }
    __syncthreads();
    if (set != 0) return;
    for (uint32_t k = 1; k < sets; ++k) {
        const float *pw = part[k * lanes + tl];
        const float m_new = fmaxf(m, pw[0]);
        const float a = exp2f(m - m_new), b = exp2f(pw[0] - m_new);
        l = l * a + pw[1] * b;
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) acc[e] = acc[e] * a + pw[2 + e] * b;
        m = m_new;
    }
    write(d, m, l, acc);
}

// The latent body's records (scaled fp16, SGLKV_ATTN_HPAD): the merge
// above with o_s = a_s y_s, the weight of split s being 2^(m_s - m*) a_s.
// A workgroup is one (query, head), of blockDim.x / 64 waves (the host
// gives 1 to 4, one per group of eight splits up to four groups): wave w
// merges groups w, w + W, ... of the splits, then wave 0 merges the waves'
// partial (m, l, o) through LDS, so a query with many splits waits for one
// memory latency per W groups, not per group (a query whose splits fit one
// group takes wave 0 alone). Workgroups are handed to the
// eight XCDs in turn (workgroup b to XCD b % 8), and g, the group of eight
// adjacent heads 8k .. 8k+7 of a query (g = query * ceil(heads / 8) + k),
// takes workgroups 64 (g / 8) + 8 m + g % 8 for m < 8: one XCD, so the
// eight (m, l, a) of a split, which share a line, are fetched into one L2
// once. Lane t handles dims 8t .. 8t+7 (+512 ...), one 16-byte read per
// split's y row (rows of whole 128-byte lines; dims past dv read the row's
// padding and are not written).
extern "C" __global__ __launch_bounds__(256) void sglkv_paged_attention_combine_h(sglkv_attn_params p) {
    __shared__ float part[3][64][10];  // waves 1..3: m, l, o[8] per lane
    const uint32_t groups = (p.query_heads + 7) / 8;
    const uint64_t t = blockIdx.x / 8;
    const uint64_t g = 8 * (t / 8) + blockIdx.x % 8;
    if (g >= p.query_count * groups) return;  // uniform over the workgroup
    const uint64_t q = g / groups;
    const uint32_t head = 8 * static_cast<uint32_t>(g % groups) + static_cast<uint32_t>(t % 8);
    if (head >= p.query_heads) return;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    uint64_t start = 0, len = 0;
    if (!attn_metadata(p, q, false, &start, &len)) return;
    const uint32_t used = static_cast<uint32_t>((len + p.chunk_tokens - 1) / p.chunk_tokens);
    // One group of splits (a short sequence): wave 0 alone, no merge (the
    // condition is the same for every wave of the workgroup).
    if (used <= 8 && wave != 0) return;
    const uint32_t nw = used <= 8 ? 1 : waves;
    const uint64_t i0 = (q * p.query_heads + head) * p.splits;
    const float4 *mla = reinterpret_cast<const float4 *>(attn_rec_mla(p, q, 0, head));
    const uint64_t mla_split = p.query_heads;  // float4s from one split's (m, l, a) to the next's
    const uint16_t *y = attn_rec_y(p, i0);
    const uint32_t hpad = SGLKV_ATTN_HPAD(p.dv);
    uint16_t *out = p.output + (q * p.query_heads + head) * p.dv;
    // Every lane of every wave runs the same iterations (the barriers below
    // need that); a lane past the row loads element 0 and stores nothing.
    for (uint32_t d0 = 0; d0 < p.dv; d0 += 512) {
        const bool active = d0 + 8 * lane < p.dv;
        const uint32_t d = active ? d0 + 8 * lane : 0;
        float m = -3.402823466e+38f, l = 0.0f;
        float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t s0 = 8 * wave; s0 < used; s0 += 8 * nw) {
            float4 r[8];
            sglkv_u16x8 v[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) {
                const uint32_t s = s0 + j < used ? s0 + j : used - 1;
                r[j] = mla[s * mla_split];
                v[j] = *reinterpret_cast<const sglkv_u16x8 *>(y + s * hpad + d);
            }
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) {
                const bool ok = s0 + j < used;
                const float m_new = ok ? fmaxf(m, r[j].x) : m;
                const float a = exp2f(m - m_new);
                const float w = ok ? exp2f(r[j].x - m_new) : 0.0f;
                l = l * a + w * r[j].y;
                const float wy = w * r[j].z;
#pragma unroll
                for (uint32_t e = 0; e < 8; ++e) {
                    // (the element copied out first: hipcc bit-casts a
                    // vector element operand as element 0)
                    const uint16_t bits = v[j][e];
                    acc[e] = acc[e] * a + wy * static_cast<float>(__builtin_bit_cast(_Float16, bits));
                }
                m = m_new;
            }
        }
        if (nw > 1) {
            // A wave with no group keeps m = -FLT_MAX, l = 0, o = 0, which
            // the merge weighs 0.
            if (wave > 0) {
                float *pw = part[wave - 1][lane];
                pw[0] = m;
                pw[1] = l;
#pragma unroll
                for (uint32_t e = 0; e < 8; ++e) pw[2 + e] = acc[e];
            }
            __syncthreads();
            if (wave == 0) {
                for (uint32_t w = 1; w < nw; ++w) {
                    const float *pw = part[w - 1][lane];
                    const float m_new = fmaxf(m, pw[0]);
                    const float a = exp2f(m - m_new), b = exp2f(pw[0] - m_new);
                    l = l * a + pw[1] * b;
#pragma unroll
                    for (uint32_t e = 0; e < 8; ++e) acc[e] = acc[e] * a + pw[2 + e] * b;
                    m = m_new;
                }
            }
            __syncthreads();
        }
        if (wave != 0 || !active) continue;
        const float linv = 1.0f / l;
        sglkv_u16x8 o8;
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) o8[e] = attn_to_bf16(acc[e] * linv);
        if (d + 8 <= p.dv && (reinterpret_cast<uintptr_t>(out + d) & 15u) == 0) {
            *reinterpret_cast<sglkv_u16x8 *>(out + d) = o8;
        } else {
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e)
                if (d + e < p.dv) out[d + e] = o8[e];
        }
    }
}
