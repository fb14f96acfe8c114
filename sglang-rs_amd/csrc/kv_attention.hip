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
// Metadata errors set the device error word (SGLKV_FLAG_ATTN_*) and skip
// the query, as the reference's kernel does.

typedef __bf16 sglkv_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sglkv_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short sglkv_u16x8 __attribute__((ext_vector_type(8)));

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

template <bool VEC>
__device__ __forceinline__ void attn_body(const sglkv_attn_params &p) {
    extern __shared__ __attribute__((aligned(16))) uint16_t attn_lds[];
    const uint32_t lane = threadIdx.x;
    const uint32_t g = lane >> 4, r = lane & 15;

    uint64_t bx = blockIdx.x;
    const uint32_t dblk = static_cast<uint32_t>(bx % p.dv_blocks);
    bx /= p.dv_blocks;
    const uint32_t hg = static_cast<uint32_t>(bx % p.head_groups);
    bx /= p.head_groups;
    const uint32_t kvh = static_cast<uint32_t>(bx % p.kv_heads);
    const uint64_t q = bx / p.kv_heads;
    const uint32_t split = blockIdx.y;

    uint64_t start = 0, len = 0;
    const bool report = lane == 0 && split == 0 && hg == 0 && dblk == 0 && kvh == 0;
    if (!attn_metadata(p, q, report, &start, &len)) return;
    const uint64_t t0 = static_cast<uint64_t>(split) * p.chunk_tokens;
    if (t0 >= len) return;
    const uint64_t t1 = len < t0 + p.chunk_tokens ? len : t0 + p.chunk_tokens;

    const uint32_t h0 = kvh * p.group + hg * SGLKV_ATTN_HEADS;
    const uint32_t nh = p.group - hg * SGLKV_ATTN_HEADS < SGLKV_ATTN_HEADS
                            ? p.group - hg * SGLKV_ATTN_HEADS
                            : SGLKV_ATTN_HEADS;
    const uint32_t d0 = dblk * SGLKV_ATTN_DV;  // first value dim of this workgroup

    // Queries of the head group, zero-padded to 16 heads x dk_pad dims; a
    // row is dk_pad + 8 elements so the 16 rows start in different banks.
    const uint32_t qstride = p.dk_pad + 8;
    uint16_t *qs = attn_lds;
    uint16_t *vt = attn_lds + SGLKV_ATTN_HEADS * qstride;
    for (uint32_t i = lane; i < SGLKV_ATTN_HEADS * p.dk_pad; i += 64) {
        const uint32_t h = i / p.dk_pad, d = i % p.dk_pad;
        uint16_t v = 0;
        if (h < nh && d < p.dk) v = p.queries[(q * p.query_heads + h0 + h) * p.dk + d];
        qs[h * qstride + d] = v;
    }
    __syncthreads();

    const uint64_t pool = reinterpret_cast<uint64_t>(p.pool);
    const uint64_t kbase = pool + p.key_offset + kvh * p.key_head_stride;
    const uint64_t vbase = pool + p.value_offset + kvh * p.value_head_stride;

    float m_run = -3.402823466e+38f;  // running max (log2 units) of head r
    float l_part = 0.0f;              // this lane's share of head r's sum
    sglkv_f32x4 o[SGLKV_ATTN_DV / 16];
#pragma unroll
    for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j) o[j] = sglkv_f32x4{0.f, 0.f, 0.f, 0.f};

    for (uint64_t tb = t0; tb < t1; tb += SGLKV_ATTN_TOKENS) {
        // Row r of score block b is token tb + 8*(r/4) + 4*b + r%4, so that
        // after the q.k product lane (g, r) holds tokens tb + 8g .. 8g+7 of
        // head r: the A-operand layout of the p.v product.
        uint64_t krow[2], vrow[2];
        bool valid[2];
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b) {
            const uint64_t tok = tb + 8 * (r >> 2) + 4 * b + (r & 3);
            bool ok = tok < t1;
            uint64_t slot = 0;
            if (ok) {
                slot = p.sequence_slots[start + tok];
                if (slot >= p.slot_count) {
                    atomicOr(p.flag, SGLKV_FLAG_ATTN_SLOT);
                    ok = false;
                    slot = 0;
                }
            }
            const uint64_t page = slot / p.page_size, pos = slot % p.page_size;
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
                vpiece[b][s] = attn_load8<VEC>(vrow[b], d0 + 8 * (g + 4 * s), p.dv, valid[b]);

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

        // Online softmax for head r over this lane's 8 tokens.
        const uint64_t vb0 = __ballot(valid[0]), vb1 = __ballot(valid[1]);
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
        const float m_new = fmaxf(m_run, mx);
        const float alpha = exp2f(m_run - m_new);
        sglkv_u16x8 pbits;
        float psum = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const float pi = exp2f(x[i] - m_new);
            psum += pi;
            pbits[i] = attn_to_bf16(pi);
        }
        l_part = l_part * alpha + psum;
        m_run = m_new;

        // Output rows are heads 4g+e: fetch their rescale factors.
        float arow[4];
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) arow[e] = __shfl(alpha, 4 * g + e);
#pragma unroll
        for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j)
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) o[j][e] *= arow[e];

        __builtin_amdgcn_wave_barrier();
        // o[head 4g+e][dim 16j + r] += sum_t p[head][t] * v[t][dim].
#pragma unroll
        for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j) {
            if (d0 + 16 * j >= p.dv) break;
            const sglkv_u16x8 vv =
                *reinterpret_cast<const sglkv_u16x8 *>(vt + (16 * j + r) * SGLKV_ATTN_VT_STRIDE + 8 * g);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(attn_as_bf16(pbits), attn_as_bf16(vv), o[j], 0,
                                                           0, 0);
        }
        __builtin_amdgcn_wave_barrier();
    }

    float l_tot = l_part + __shfl_xor(l_part, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (p.splits == 1) {
        float linv[4];
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) linv[e] = 1.0f / __shfl(l_tot, 4 * g + e);
#pragma unroll
        for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j) {
            const uint32_t dim = d0 + 16 * j + r;
            if (dim >= p.dv) continue;
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) {
                const uint32_t h = 4 * g + e;
                if (h < nh)
                    p.output[(q * p.query_heads + h0 + h) * p.dv + dim] = attn_to_bf16(o[j][e] * linv[e]);
            }
        }
    } else {
        // Partial record of (query, head, split): [m, l, o[0..dv)].
        const uint64_t rec = p.dv + 2;
        if (dblk == 0 && g == 0 && r < nh) {
            float *pr = p.partial + ((q * p.query_heads + h0 + r) * p.splits + split) * rec;
            pr[0] = m_run;
            pr[1] = l_tot;
        }
#pragma unroll
        for (uint32_t j = 0; j < SGLKV_ATTN_DV / 16; ++j) {
            const uint32_t dim = d0 + 16 * j + r;
            if (dim >= p.dv) continue;
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) {
                const uint32_t h = 4 * g + e;
                if (h < nh) p.partial[((q * p.query_heads + h0 + h) * p.splits + split) * rec + 2 + dim] = o[j][e];
            }
        }
    }
}

}  // namespace

extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_v16(sglkv_attn_params p) {
    attn_body<true>(p);
}

extern "C" __global__ __launch_bounds__(64) void sglkv_paged_attention_v2(sglkv_attn_params p) {
    attn_body<false>(p);
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
