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
//    tokens 8*(l/16)..+7); V is transposed through LDS into the B layout;
//  - long sequences are split over gridDim.y (flash-decoding): each split
//    writes (max, sum, unnormalised output) and a combine kernel merges
//    them, so a small batch still fills 256 CUs.
// Two bodies share this math. The pipelined one (head dims up to 128,
// 16-byte rows, power-of-two pages: every Llama/Qwen-style decode) loads
// the slots of block i+2 and the K/V rows of block i+1 while it computes
// block i, so a wave never waits on the dependent slot -> row loads; the
// generic one serves every other shape (MLA widths, odd dims) one block at
// a time.
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
    if (!valid) return v;
    if (VEC) {
        if (dim < limit)
            v = *reinterpret_cast<__attribute__((address_space(1))) const sglkv_u16x8 *>(row + 2ull * dim);
    } else {
        const __attribute__((address_space(1))) uint16_t *p =
            reinterpret_cast<__attribute__((address_space(1))) const uint16_t *>(row);
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e)
            if (dim + e < limit) v[e] = p[dim + e];
    }
    return v;
}

__device__ __forceinline__ uint16_t attn_to_bf16(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
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
struct attn_state {
    float m_run;   // running max (log2 units) of head r
    float l_part;  // this lane's share of head r's sum
    sglkv_f32x4 o[SGLKV_ATTN_DV / 16];
};

__device__ __forceinline__ void attn_state_init(attn_state &st) {
    st.m_run = -3.402823466e+38f;
    st.l_part = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j) st.o[j] = sglkv_f32x4{0.f, 0.f, 0.f, 0.f};
}

// One 32-token block after q.k: sc[b][e] is head r's score of row 4g+e of
// score block b (token 8g + 4b + e of the block), vb0/vb1 the validity
// ballots of the rows, and vt the block's values transposed in LDS
// (vt[dim][token]). Updates the softmax state and o += p.v.
template <bool FULL_DV = false>
__device__ __forceinline__ void attn_softmax_pv(const sglkv_attn_params &p, uint32_t g, uint32_t d0,
                                                const sglkv_f32x4 (&sc)[2], uint64_t vb0, uint64_t vb1,
                                                const uint16_t *vt, uint32_t r, attn_state &st) {
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
    sglkv_u16x8 pbits;
    float psum = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        const float pi = exp2f(x[i] - m_new);
        psum += pi;
        pbits[i] = attn_to_bf16(pi);
    }
    st.l_part = st.l_part * alpha + psum;
    st.m_run = m_new;

    // Output rows are heads 4g+e: fetch their rescale factors.
    float arow[4];
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) arow[e] = __shfl(alpha, 4 * g + e);
#pragma unroll
    for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j)
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) st.o[j][e] *= arow[e];

    __builtin_amdgcn_wave_barrier();
    // o[head 4g+e][dim 16j + r] += sum_t p[head][t] * v[t][dim].
#pragma unroll
    for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j) {
        if (!FULL_DV && d0 + 16 * j >= p.dv) break;
        const sglkv_u16x8 vv =
            *reinterpret_cast<const sglkv_u16x8 *>(vt + (16 * j + r) * SGLKV_ATTN_VT_STRIDE + 8 * g);
        st.o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(pbits), attn_as_bf16(vv), st.o[j], 0,
                                                          0, 0);
    }
    __builtin_amdgcn_wave_barrier();
}

// Output (one split) or the split record [m, l, o[0..dv)].
__device__ __forceinline__ void attn_finish(const sglkv_attn_params &p, const attn_work &w, uint32_t g,
                                            uint32_t r, const attn_state &st) {
    float l_tot = st.l_part + __shfl_xor(st.l_part, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (p.splits == 1) {
        float linv[4];
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) linv[e] = 1.0f / __shfl(l_tot, 4 * g + e);
#pragma unroll
        for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j) {
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
        const uint64_t rec = p.dv + 2;
        if (w.dblk == 0 && g == 0 && r < w.nh) {
            float *pr = p.partial + ((w.q * p.query_heads + w.h0 + r) * p.splits + w.split) * rec;
            pr[0] = st.m_run;
            pr[1] = l_tot;
        }
#pragma unroll
        for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j) {
            const uint32_t dim = w.d0 + 16 * j + r;
            if (dim >= p.dv) continue;
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) {
                const uint32_t h = 4 * g + e;
                if (h < w.nh)
                    p.partial[((w.q * p.query_heads + w.h0 + h) * p.splits + w.split) * rec + 2 + dim] =
                        st.o[j][e];
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
        // Value pieces first, so their loads are in flight during q.k: lane
        // (g, r) loads dims d0 + 8*(g + 4s) .. +7 of its two tokens.
        sglkv_u16x8 vpiece[2][4];
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b)
#pragma unroll
            for (uint32_t s = 0; s < 4; ++s)
                vpiece[b][s] = attn_load8<VEC>(vrow[b], w.d0 + 8 * (g + 4 * s), p.dv, valid[b]);

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

}  // namespace

extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_v16(sglkv_attn_params p) {
    attn_body<true>(p);
}

extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_v2(sglkv_attn_params p) {
    attn_body<false>(p);
}

// Head dims exactly 128 (no per-dim masks) / up to 128.
extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_pipe128(sglkv_attn_params p) {
    attn_pipe_body<true>(p);
}

extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_pipe(sglkv_attn_params p) {
    attn_pipe_body<false>(p);
}

// Merges the split records of one (query, head): m* = max m_s,
// out = sum_s 2^(m_s - m*) o_s / sum_s 2^(m_s - m*) l_s.
extern "C" __global__ __launch_bounds__(128) void sglkv_paged_attention_combine(sglkv_attn_params p) {
    const uint64_t q = blockIdx.x / p.query_heads;
    const uint32_t head = static_cast<uint32_t>(blockIdx.x % p.query_heads);
    uint64_t start = 0, len = 0;
    if (!attn_metadata(p, q, false, &start, &len)) return;
    const uint64_t used = (len + p.chunk_tokens - 1) / p.chunk_tokens;
    const uint64_t rec = p.dv + 2;
    const float *base = p.partial + (q * p.query_heads + head) * p.splits * rec;
    float m = -3.402823466e+38f;
    for (uint64_t s = 0; s < used; ++s) m = fmaxf(m, base[s * rec]);
    float l = 0.0f;
    for (uint64_t s = 0; s < used; ++s) l += exp2f(base[s * rec] - m) * base[s * rec + 1];
    const float linv = 1.0f / l;
    for (uint32_t d = threadIdx.x; d < p.dv; d += 128) {
        float acc = 0.0f;
        for (uint64_t s = 0; s < used; ++s) acc += exp2f(base[s * rec] - m) * base[s * rec + 2 + d];
        p.output[(q * p.query_heads + head) * p.dv + d] = attn_to_bf16(acc * linv);
    }
}
