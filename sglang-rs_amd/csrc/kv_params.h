/*
 * kv_params.h -- launch parameters shared by the host launcher
 * (kv_runtime.cpp) and the gfx950 kernels (kv_kernels.hip).
 *
 * Every copy on this path moves whole "rows": the bytes one token owns in
 * one layer for each of its tensors (K and V, or the single MLA latent row).
 * A copy has a source side and a destination side, each of one of two kinds:
 *
 *  ROWS  contiguous transfer rows: row r of tensor t starts at
 *        plane[t] + r * stride[t]; the row is token-major (heads then dim).
 *  POOL  one layer of a page-major pool: row r lives in physical slot
 *        slots[r]; page = slot / page_size, pos = slot % page_size and the
 *        row's tensor-t bytes start at
 *            plane[t] + page * stride + pos * pos_mult
 *        where plane[t] already includes the layer's in-page tensor offset
 *        (PagedKvCacheLayout::tensor_token_byte_range,
 *        crates/sglang-srt/src/kv_cache.rs:653-700). Head chunk h of the row
 *        sits head_stride bytes after chunk h-1: NHD pages keep the row
 *        contiguous (head_stride = chunk bytes, pos_mult = row bytes), HND
 *        pages put each head's page_size chunks together (head_stride =
 *        page_size * chunk bytes, pos_mult = chunk bytes).
 *
 * A launch covers one layer per gridDim.y: layer y's planes sit
 * y * layer_stride bytes after layer 0's on each side (row offsets do not
 * depend on the layer).
 *
 * Vectors: the host picks the widest access width VB in {16, 8, 4, 2, 1}
 * that divides every base, stride and chunk size, so every access is
 * naturally aligned. Sizes below are in units of VB.
 */
#ifndef SGLKV_PARAMS_H
#define SGLKV_PARAMS_H

#include <stdint.h>

#define SGLKV_SIDE_ROWS 0u
#define SGLKV_SIDE_POOL 1u

/* Threads per workgroup. */
#define SGLKV_BLOCK_THREADS 256u
/* Largest row tile one workgroup stages, and the rows each thread keeps in
 * flight (loads issued before the stores). The code object exports the
 * values it was built with (sglkv_max_tile_rows, sglkv_rows_per_thread);
 * the launcher reads them at load time and sizes its tiles from them. */
#ifndef SGLKV_MAX_TILE_ROWS
#define SGLKV_MAX_TILE_ROWS 512u
#endif
#ifndef SGLKV_ROWS_PER_THREAD
#define SGLKV_ROWS_PER_THREAD 8u
#endif

/* Bits of the device error word. */
#define SGLKV_FLAG_SLOT 1u /* a slot map entry >= slot_count (reference flag value) */
#define SGLKV_FLAG_PAGE 2u /* a page-table entry out of range while resolving spans */
#define SGLKV_FLAG_SPAN 4u /* a row not covered by any span */
#define SGLKV_FLAG_REQUEST 8u /* a page request outside its source or target region */
/* Paged attention metadata errors (the reference kernel's flag values 1, 2
 * and 4, cuda_attention.rs:64-98, shifted above the copy flags). */
#define SGLKV_FLAG_ATTN_REQUEST 16u  /* query_request_indices entry >= request_count */
#define SGLKV_FLAG_ATTN_SEQUENCE 32u /* request range or query length invalid */
#define SGLKV_FLAG_ATTN_SLOT 64u     /* a sequence slot >= slot_count */

/* A resolved row offset that must not be touched. */
#define SGLKV_INVALID_OFFSET 0xFFFFFFFFFFFFFFFFull

typedef struct sglkv_side {
    uint64_t plane[2];      /* byte address of tensor t's data (see above) */
    uint64_t stride[2];     /* ROWS: row stride of tensor t; POOL: page stride (both) */
    const uint64_t *slots;  /* POOL: physical slot of each row */
    uint64_t pos_mult[2];   /* POOL: bytes between adjacent in-page positions of tensor t */
    uint64_t head_stride[2];/* bytes between head chunks of one row of tensor t */
    uint64_t slot_count;    /* POOL: valid slots are [0, slot_count) */
    uint64_t layer_stride;  /* bytes between consecutive layers' data (blockIdx.y = layer) */
    uint32_t page_size;     /* POOL: tokens per page */
    uint32_t reserved;
} sglkv_side;

/* The two tensors of a row may differ in width (MLA's 576/512-dim pair):
 * tensor 0 owns the row's first vpt vectors, tensor 1 the remaining
 * vpr - vpt, and each tensor's row is cut into head chunks of vpc[t]
 * vectors. */
typedef struct sglkv_copy_params {
    sglkv_side src;
    sglkv_side dst;
    uint32_t *flag;         /* device error word (OR of SGLKV_FLAG_*) */
    float *scale_src;       /* optional per-layer scales copied bit-exactly; layer y's */
    float *scale_dst;       /* scale_count floats follow layer y - 1's */
    uint32_t scale_count;   /* floats to copy per layer (0: none) */
    uint32_t rows;          /* rows in this launch */
    uint32_t vpr;           /* vectors per row, all tensors */
    uint32_t vpt;           /* vectors of tensor 0's row */
    uint32_t vpc[2];        /* vectors per head chunk of tensor t */
    uint32_t tile_rows;     /* rows per workgroup = blockDim.y * rows per thread */
    uint32_t line_rows;     /* > 1: head-major pages with head chunks of 128 / line_rows
                               bytes; lanes regrouped so that line_rows consecutive rows
                               of one chunk (one cache line of a page) share a wave
                               (blockDim.x == vpr, blockDim.y % line_rows == 0) */
} sglkv_copy_params;

/* Byte-realigning copy: for rows whose chunks are not whole 16-byte vectors
 * at 16-byte aligned addresses (packed-MLA rows of 649 bytes, odd row
 * strides), every memory access is still an aligned 16-byte vector.
 * Segment (t, h) of a row is head chunk h of tensor t: chunk[t] bytes from
 * source address S to destination address D. The workgroup loads the
 * aligned 16-byte vectors covering [S, S + chunk) into LDS (seg[t] vectors
 * reserved per segment, enough for any alignment), then builds each
 * aligned destination vector of [D, D + chunk) from LDS shifted by
 * (S - D) mod 16 and stores it; the partial first and last vectors are
 * written as aligned 8/4/2/1-byte pieces. A row occupies vrow LDS vectors:
 * tensor 0's heads[0] segments (vt0 vectors), then tensor 1's. */
typedef struct sglkv_realign_params {
    sglkv_side src;
    sglkv_side dst;
    uint32_t *flag;
    float *scale_src;
    float *scale_dst;
    uint32_t scale_count;
    uint32_t rows;
    uint32_t chunk[2];      /* bytes per segment of tensor t */
    uint32_t seg[2];        /* LDS vectors per segment of tensor t: (chunk + 30) / 16 */
    uint32_t vt0;           /* LDS vectors of tensor 0's segments */
    uint32_t vrow;          /* LDS vectors per row */
    uint32_t tile_rows;     /* rows per workgroup = blockDim.y * rows per thread */
    uint32_t rows_per_thread;
    const uint8_t *zero;    /* 16 readable bytes (the context's zero row): the load of lanes
                               with nothing to load */
} sglkv_realign_params;

/* Realigning kernel limits: rows a thread keeps in flight (the code object
 * exports the value it was built with, sglkv_realign_rows_per_thread, and
 * the launcher sizes tiles from it), and the widest row it takes (rows
 * wider than SGLKV_REALIGN_MAX_ROW_VECTORS LDS vectors use the plain
 * kernels with narrower accesses). The LDS buffer carries 16 bytes of
 * padding before the first row and SGLKV_REALIGN_TAIL_PAD after the last,
 * so that the shifted reads of the first and last vectors stay inside it. */
#ifndef SGLKV_REALIGN_ROWS_PER_THREAD
#define SGLKV_REALIGN_ROWS_PER_THREAD 4u  /* measured on MI355X (649-byte rows): 4 over 2, 8, 16 */
#endif
#define SGLKV_REALIGN_MAX_ROW_VECTORS 256u
#define SGLKV_REALIGN_TAIL_PAD 32u
/* Dynamic LDS of a realigning workgroup: the tile's staged row offsets
 * (one per tensor and side), the front pad, the rows and the tail pad. */
#define SGLKV_REALIGN_LDS_BYTES(tile_rows, vrow)                                                   \
    (32u * (tile_rows) + 16u + 16u * (tile_rows) * (vrow) + SGLKV_REALIGN_TAIL_PAD)

/* One request's run of rows (KvCacheTransferSpan,
 * crates/sglang-srt/src/transfer.rs:495-505): rows [row_start, row_start +
 * token_count) hold request tokens [token_offset, token_offset +
 * token_count); token k is in page page_table[page_table_start + k /
 * page_size] at position k % page_size. */
typedef struct sglkv_span {
    uint32_t row_start;
    uint32_t token_offset;
    uint32_t token_count;
    uint32_t page_table_start;
} sglkv_span;

typedef struct sglkv_resolve_params {
    const sglkv_span *spans;  /* sorted by row_start, non-overlapping */
    const int32_t *page_table;
    uint64_t *out_slots;      /* one slot per row; SGLKV_INVALID_OFFSET on failure */
    uint32_t *flag;
    uint64_t page_table_len;
    uint64_t page_count;      /* pages of the pool the table indexes */
    uint32_t span_count;
    uint32_t page_size;
    uint32_t rows;
    uint32_t reserved;
} sglkv_resolve_params;

/* Page-request execution: request i copies length_i bytes from source_i to
 * target_base + target_offset_i. Workgroup b handles chunk b % chunks of
 * request b / chunks (chunk = SGLKV_REQUEST_CHUNK bytes). */
#define SGLKV_REQUEST_CHUNK 65536u

typedef struct sglkv_request {
    uint64_t source;
    uint64_t target_offset;
    uint64_t length;
} sglkv_request;

typedef struct sglkv_request_params {
    const sglkv_request *requests;
    uint32_t *flag;
    uint64_t count;
    uint64_t chunks;        /* chunks per request (of the longest request) */
    uint64_t target_base;   /* added to every target_offset (0: offsets are addresses) */
    uint64_t source_lo, source_hi;   /* allowed source bytes [lo, hi) */
    uint64_t target_lo, target_hi;   /* allowed target bytes [lo, hi) */
} sglkv_request_params;

/* Paged decode/prefill attention over bf16 K/V pages.
 *
 * Query q attends the first len_q = query_sequence_lengths[q] slots of its
 * request's slot list (sequence_slots[request_slot_offsets[r] ..]). Key k of
 * KV head h at slot s is at
 *     pool + (s / page_size) * page_stride + key_offset
 *          + h * key_head_stride + (s % page_size) * key_token_stride
 * (NHD: head stride = Dk * 2, token stride = key row bytes; HND: head
 * stride = page_size * Dk * 2, token stride = Dk * 2), values alike.
 *
 * A workgroup is one wave and owns (query, KV head, group of up to
 * SGLKV_ATTN_HEADS query heads, block of SGLKV_ATTN_DV value dims) for the
 * tokens [split * chunk_tokens, +chunk_tokens) of gridDim.y's split. With
 * one split it writes the output; otherwise it writes a partial record
 * (running max m in log2 units, sum l, unnormalised o[dv]; the layout of
 * SGLKV_ATTN_OPAD) that the combine kernel merges. */
#define SGLKV_ATTN_TOKENS 32u   /* tokens per wave iteration */
#define SGLKV_ATTN_HEADS 16u    /* query heads per workgroup (MFMA N) */
#define SGLKV_ATTN_DV 128u      /* value dims per workgroup */
#define SGLKV_ATTN_VT_STRIDE 40u /* u16 per transposed-V row in LDS (32 tokens + pad) */
#define SGLKV_ATTN_MAX_DK 1024u /* query/key head dim limit (LDS-resident queries) */
/* Split records: record i = (query * query_heads + head) * splits + split
 * keeps its unnormalised o[dv] at partial + i * SGLKV_ATTN_OPAD(dv) floats
 * (rows padded to whole 128-byte lines, so that the writes fill every line
 * they touch) and its m, l at partial + records * SGLKV_ATTN_OPAD(dv) + 2 i. */
#define SGLKV_ATTN_OPAD(dv) (((dv) + 31u) & ~31u)
/* The latent body's split records are scaled fp16: record i keeps
 * y[dv] = o / a at partial + i * SGLKV_ATTN_HPAD(dv) halves (rows of whole
 * 128-byte lines), a = max |o| over the record (so |y| <= 1), and
 * (m, l, a, 0) as four floats at partial + records * SGLKV_ATTN_HPAD(dv)
 * halves + 16 j bytes, j = (query * splits + split) * query_heads + head
 * (a split's heads adjacent). sglkv_paged_attention_combine_h merges them. */
#define SGLKV_ATTN_HPAD(dv) (((dv) + 63u) & ~63u)
/* The wide bodies (many query heads per KV head, e.g. MLA): a workgroup of
 * SGLKV_ATTN_WIDE_WAVES waves serves SGLKV_ATTN_WIDE_GROUPS groups of
 * SGLKV_ATTN_HEADS heads, two waves per group; K dims padded to 32*DKC, V
 * dims to 16*NJ. Its LDS: one 32-token block (K rows of 32*DKC+8 and V rows
 * of 16*NJ+16 u16), a 2 KiB partial score tile per wave, the chunk's slot
 * table (u32, at most SGLKV_ATTN_WIDE_SLOTS tokens, which bounds the chunk)
 * and a flag. */
#define SGLKV_ATTN_WIDE_GROUPS 4u
#define SGLKV_ATTN_WIDE_WAVES 8u
#define SGLKV_ATTN_WIDE_SLOTS 4096u
#define SGLKV_ATTN_WIDE_LDS_BYTES(DKC, NJ)                                                     \
    (2u * SGLKV_ATTN_TOKENS * ((32u * (DKC) + 8u) + (16u * (NJ) + 16u)) +                      \
     SGLKV_ATTN_WIDE_WAVES * 2u * 64u * 16u + 4u * SGLKV_ATTN_WIDE_SLOTS + 16u)
/* The latent body (MLA decode: K rows up to 576 dims, V rows up to 512): a
 * workgroup of SGLKV_ATTN_LATENT_WAVES waves serves up to
 * SGLKV_ATTN_LATENT_HEADS query heads of one KV head, 32 per wave. Its LDS:
 * two stages of a 32-token block's K rows (dims [0, 512) at a pitch of 1,040
 * bytes, dims [512, 576) as 128-byte rows) and two of its V rows (pitch
 * 1,088 bytes), the chunk's slot table and a flag. */
#define SGLKV_ATTN_LATENT_WAVES 4u
#define SGLKV_ATTN_LATENT_HEADS 128u
#define SGLKV_ATTN_LATENT_KSTAGE (SGLKV_ATTN_TOKENS * (1040u + 128u))
#define SGLKV_ATTN_LATENT_VSTAGE (SGLKV_ATTN_TOKENS * 1088u)
#define SGLKV_ATTN_LATENT_LDS_BYTES                                                            \
    (2u * (SGLKV_ATTN_LATENT_KSTAGE + SGLKV_ATTN_LATENT_VSTAGE) + 4u * SGLKV_ATTN_WIDE_SLOTS + 16u)
/* The staged bodies (K and V head dims d = 64, 128 or 256, at most
 * SGLKV_ATTN_HEADS query heads per KV head): one wave per workgroup,
 * SGLKV_ATTN_STAGED_STAGES LDS stages of a 32-token block (64 d bytes of K
 * rows, then as many of V rows) and the chunk's slot table (at most
 * SGLKV_ATTN_STAGED_SLOTS tokens, which bounds the chunk). */
#define SGLKV_ATTN_STAGED_STAGES 2u
#define SGLKV_ATTN_STAGED_SLOTS 1024u
#define SGLKV_ATTN_STAGED_LDS_BYTES(d) (SGLKV_ATTN_STAGED_STAGES * 128u * (d) + 4u * SGLKV_ATTN_STAGED_SLOTS)
/* The dims-128 staged body keeps K in registers: two stages of V rows only
 * (64 d bytes each) and the slot table. */
#define SGLKV_ATTN_KREG_LDS_BYTES(d) (SGLKV_ATTN_STAGED_STAGES * 64u * (d) + 4u * SGLKV_ATTN_STAGED_SLOTS)

typedef struct sglkv_attn_params {
    const uint16_t *queries;              /* bf16 [query][query_head][dk] */
    const uint32_t *query_request_indices;
    const uint64_t *query_sequence_lengths;
    const uint64_t *request_slot_offsets; /* request_count + 1 */
    const uint64_t *sequence_slots;
    const uint8_t *pool;
    uint16_t *output;                     /* bf16 [query][query_head][dv] */
    float *partial;                       /* split records, or null */
    uint32_t *flag;
    uint64_t query_count;
    uint64_t request_count;
    uint64_t sequence_slot_count;
    uint64_t slot_count;
    uint64_t page_size;
    uint64_t page_stride;
    uint64_t key_offset, value_offset;
    uint64_t key_head_stride, key_token_stride;
    uint64_t value_head_stride, value_token_stride;
    uint64_t chunk_tokens;                /* tokens per split */
    uint32_t query_heads, kv_heads;
    uint32_t group;                       /* query heads per KV head */
    uint32_t head_groups;                 /* ceil(group / SGLKV_ATTN_HEADS) */
    uint32_t dk, dk_pad;                  /* dk_pad = dk rounded up to 32 */
    uint32_t dv, dv_blocks;               /* dv_blocks = ceil(dv / SGLKV_ATTN_DV) */
    uint32_t splits;
    uint32_t page_shift;                  /* log2(page_size) if a power of two, else 32 */
    float scale_log2;                     /* scale * log2(e) */
    float reserved_f;
    /* Pipelined body only (page size a power of two, strides < 2^32): */
    const uint8_t *zero_row;              /* SGLKV_ZERO_ROW_BYTES of zeros (context-owned) */
    uint32_t page_stride32;
    uint32_t key_token_stride32, value_token_stride32;
    uint32_t reserved2;
} sglkv_attn_params;

/* Both tensors of one layer for `count` slots in one launch (key and value
 * rows of unequal width, as MLA writes them): thread t moves piece
 * t % (pieces[0] + pieces[1]) of row t / (pieces[0] + pieces[1]), the key
 * row's pieces first. A piece is W bytes (kernel variant: 16 or 1). */
typedef struct sglkv_pair_slots_params {
    const uint64_t *slots;
    uint64_t count;
    uint64_t slot_count;
    uint8_t *pool;
    uint64_t page_size;
    uint64_t page_stride;
    uint64_t offset[2];      /* in-page offset of the layer's key / value region */
    uint64_t row_bytes[2];
    const uint8_t *rows[2];  /* source rows of each tensor */
    uint64_t row_stride[2];
    uint64_t pieces[2];      /* row_bytes / W */
    uint32_t *flag;          /* device error word (SGLKV_FLAG_SLOT) */
    uint32_t reserved;
} sglkv_pair_slots_params;

/* Bytes of zeros the context keeps for reads that must contribute nothing
 * (>= the widest row piece a pipelined attention lane reads, 256 B). */
#define SGLKV_ZERO_ROW_BYTES 1024u

#endif
