/*
 * ekv_kernels.h - hot-path HIP kernels of the sparse-KV residency path (gfx950).
 *
 * Every entry point validates shapes on the host, launches asynchronously on
 * the HIP stream passed by the caller (NULL = the legacy default stream), and
 * returns 0, or -1 with a message for ev_error() (declared in elastic_vmm.h).
 * No entry point allocates device memory or synchronizes the stream.
 * Tensors are described by plain pointers, dtype codes, shapes and element
 * strides; nothing here depends on PyTorch.
 */
#ifndef EKV_KERNELS_H
#define EKV_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types understood by ekv_tensor. Index tensors must be INT32/INT64. */
enum ekv_dtype {
    EKV_INT32 = 1,
    EKV_INT64 = 2,
    EKV_UINT8 = 3,
    EKV_INT8 = 4,
    EKV_INT16 = 5,
    EKV_BFLOAT16 = 6,
    EKV_FLOAT16 = 7,
    EKV_FLOAT32 = 8,
};

/* A strided device tensor of up to 4 dimensions; strides are in elements. */
typedef struct ekv_tensor {
    void* data;
    int32_t dtype;      /* enum ekv_dtype */
    int32_t ndim;
    int64_t shape[4];
    int64_t stride[4];
} ekv_tensor;

/* A KV pool seen as planes of fixed-size rows: plane (layer l, kv) starts at
 * base + l*layer_stride + kv*kv_stride and slot s of it at + s*row_stride. */
typedef struct ekv_planes {
    void* base;
    int64_t layers;       /* layers in the pool */
    int64_t kv;           /* planes per layer: 1, or 2 for separate K and V */
    int64_t layer_stride; /* bytes */
    int64_t kv_stride;    /* bytes */
    int64_t row_stride;   /* bytes between slot s and slot s+1 */
    int64_t row_bytes;    /* payload bytes per slot row */
    int64_t rows;         /* slots per plane: a slot >= rows is out of range */
} ekv_planes;

/* Dense destination (or source) rows addressed by (layer, batch, kv, lane). */
typedef struct ekv_kv_rows {
    void* data;
    int64_t layer_stride; /* bytes */
    int64_t batch_stride; /* bytes */
    int64_t kv_stride;    /* bytes */
    int64_t lane_stride;  /* bytes */
} ekv_kv_rows;

/* ABI revision of this header; bumped on any incompatible change. */
#define EKV_ABI_VERSION 3
int ekv_abi_version(void);

/* Fingerprint (32 hex digits) of the sources the library was built from; the
 * Python loader refuses a library whose fingerprint is not the one of the
 * sources beside it. No reference counterpart. */
const char* ekv_source_hash(void);

/*
 * Resident lookup with optional miss compaction.
 * Replaces: adaptive_sparse/resident_lookup.py:29-40 (resolve_resident) and
 * its kernel :6-26; torch twin adaptive_sparse/request_residency.py:819-825.
 *
 * Shapes (L = topk.shape[0]; the reference always has L = 1):
 *   topk      [L, B, K]           int32/int64 block ids, -1 = padding
 *   table     [R, T] or [L, R, T] int32/int64
 *   mapping   NULL, [N] or [L, N] int32/int64; NULL = single level (the table
 *                                 value is the slot)
 *   rows      [B], lengths [B], selected [S]   int32/int64
 *   output    [L, B, K*block_size] int32, any strides
 *   misses    NULL or [L, B, K*block_size] int32
 *   miss_count NULL or [L, B] int32 (both NULL or both given)
 * For each selected row r = selected[i], each layer l and lane o:
 *   block = topk[l, r, o / bs], pos = block*bs + o % bs,
 *   valid = block >= 0 && pos < lengths[r],
 *   output[l, r, o] = valid ? int32(mapping[l?, table[l?, rows[r], pos]]) : -1.
 * Unselected rows are left untouched. With compaction, misses[l, r, 0:c] gets
 * the lanes o with valid && output == 0 (slot 0 = not resident) in ascending
 * order and miss_count[l, r] = c; misses[l, r, c:] is left untouched.
 * Where the reference would read out of bounds (rows[r] >= R, pos >= T, a
 * mapping index outside [0, N), a selected row outside [0, B)) the lane
 * returns -1 and is not a miss, or the row is skipped.
 */
int ekv_resolve_resident(const ekv_tensor* topk, const ekv_tensor* table,
                         const ekv_tensor* mapping, const ekv_tensor* rows,
                         const ekv_tensor* lengths, const ekv_tensor* selected,
                         const ekv_tensor* output, const ekv_tensor* misses,
                         const ekv_tensor* miss_count, int64_t block_size,
                         void* stream);

/*
 * Single-level resident lookup with a residency summary in front of the
 * table. Same contract as ekv_resolve_resident with mapping = NULL.
 * resident_bits [R, W] or [L, R, W] int32 is a bit row per table row: bit q
 * covers positions [q << bits_shift, (q + 1) << bits_shift), so
 * W >= ceil(ceil(T / 2^bits_shift) / 32). Bit q must be set whenever a
 * position it covers has table[., p] != 0; a set bit over positions that
 * are all 0 is allowed (a superset only costs table reads).
 *   bits_shift = 0: one bit per position (ekv_residency_bits keeps it exact);
 *   bits_shift = 6: one bit per 64 positions = one 128-byte line of an int16
 *   table, 1/64 of the per-position bitmap's bytes.
 * Lanes whose bit is clear return slot 0 without reading their table entry,
 * so misses in unresident groups cost one bit instead of a cache line.
 * 0 <= bits_shift <= 20.
 * No reference counterpart: an acceleration of ekv_resolve_resident
 * (adaptive_sparse/resident_lookup.py:29-40 semantics are unchanged).
 */
int ekv_resolve_resident_bits(const ekv_tensor* topk, const ekv_tensor* table,
                              const ekv_tensor* resident_bits, int64_t bits_shift,
                              const ekv_tensor* rows, const ekv_tensor* lengths,
                              const ekv_tensor* selected, const ekv_tensor* output,
                              const ekv_tensor* misses, const ekv_tensor* miss_count,
                              int64_t block_size, void* stream);

/*
 * ekv_resolve_resident (single level) over an int16 table of local slots:
 * a lane whose entry v = table[.., rows[r], pos] is >= 1 gets slot
 * slot_base[rows[r]] + v - 1, a lane with v <= 0 gets 0 (not resident);
 * invalid lanes get -1 and the miss list is as in ekv_resolve_resident.
 *   table [R, T] or [L, R, T] int16; slot_base [R] int32/int64;
 *   resident_bits as in ekv_resolve_resident_bits, or NULL.
 * Half the table bytes of the int32 global-slot form for hot buffers of up to
 * 32767 slots per request (ekv_swap_in maintains either form).
 * No reference counterpart: an acceleration of ekv_resolve_resident
 * (adaptive_sparse/resident_lookup.py:29-40 semantics are unchanged).
 */
int ekv_resolve_resident_local(const ekv_tensor* topk, const ekv_tensor* table,
                               const ekv_tensor* slot_base, const ekv_tensor* resident_bits,
                               int64_t bits_shift, const ekv_tensor* rows, const ekv_tensor* lengths,
                               const ekv_tensor* selected, const ekv_tensor* output,
                               const ekv_tensor* misses, const ekv_tensor* miss_count,
                               int64_t block_size, void* stream);

/*
 * Exact residency summary of a table (int16, int32 or int64): bit j of word
 * w of row q = 1 when any position p in [(32w + j) << bits_shift,
 * (32w + j + 1) << bits_shift) has table[.., q, p] != 0. Words
 * 0 .. ceil(ceil(T / 2^bits_shift) / 32) - 1 are written, bits past the table
 * are 0; words past them are left as they are.
 * No reference counterpart (maintenance of the summary above).
 */
int ekv_residency_bits(const ekv_tensor* table, const ekv_tensor* resident_bits,
                       int64_t bits_shift, void* stream);

/*
 * Row gather over a fixed-position virtual layout.
 * Replaces: experimental/sparse_read.py:33-51 (gather_rows) and its kernel
 * :11-30.
 *   raw [E] payload (any dtype), positions [B, S], request_ids [B],
 *   lengths [B], request_table [Q, W] (indirect only), slot_offsets [N]
 *   (indirect only), output [B, S, width] of raw's dtype.
 * valid = 0 <= pos < lengths[b]; the source element offset is
 *   direct:   sink_elements + request_ids[b]*request_stride + pos*width
 *   indirect: slot_offsets[request_table[request_ids[b], pos]]
 * and output[b, s, :] = raw[offset : offset + width], or zeros when invalid
 * (or, unlike the reference, when the row would fall outside raw).
 */
int ekv_gather_rows(const ekv_tensor* raw, const ekv_tensor* positions,
                    const ekv_tensor* request_ids, const ekv_tensor* lengths,
                    const ekv_tensor* request_table,
                    const ekv_tensor* slot_offsets, const ekv_tensor* output,
                    int64_t request_stride, int64_t sink_elements, int indirect,
                    void* stream);

/*
 * Top-K sparse KV gather from a (chunked, VMM-backed) pool of planes.
 * No reference kernel: the reference's gather is the indirect mode of
 * experimental/sparse_read.py:11-30 over one plane; this is its multi-plane
 * form for the per-layer slot lists produced by ekv_resolve_resident.
 *   slots [L, B, K] int32/int64 (stride 0 on dim 0 shares one list over layers)
 * For l < L, b < B, kv < planes->kv, k < K:
 *   out(l, b, kv, k) = plane(l, kv)[slot] if zero_below <= slot < rows,
 *                      else planes->row_bytes zero bytes.
 * zero_below = 1 makes slot 0 (the sink, "not resident") and -1 zero rows.
 */
int ekv_gather_kv(const ekv_planes* planes, const ekv_tensor* slots,
                  const ekv_kv_rows* out, int64_t zero_below, void* stream);

/*
 * Inverse of ekv_gather_kv: plane(l, kv)[slot] = src(l, b, kv, k) for every
 * slot with zero_below <= slot < rows; other lanes write nothing. Two lanes
 * naming the same slot race (the caller must pass distinct slots).
 * Replaces the byte movement of the third-party host-copy kernels used by
 * adaptive_sparse/migration.py:109-111,232-237 (unpack side).
 */
int ekv_scatter_kv(const ekv_planes* planes, const ekv_tensor* slots,
                   const ekv_kv_rows* src, int64_t zero_below, void* stream);

/* Recency stamps one LRU step spans: hits take step * 8192 + lane, misses
 * step * 8192 + 4096 + lane (a row has at most 4096 lanes), so every step's
 * stamps exceed all earlier steps' whatever the width of each call. */
#define EKV_SWAP_STEP_STAMPS 8192

/* Error bits a swap-in ORs into its status word (a row so refused changes
 * nothing and records empty promotions). */
#define EKV_SWAP_STAMP_OVERFLOW 1  /* (step + 1) * EKV_SWAP_STEP_STAMPS would reach 2^31 */
#define EKV_SWAP_SHARED_REQUEST 2  /* two selected rows name one request */

/*
 * Hot-buffer swap-in with batch-token LRU replacement, run after the lookup.
 * Policy: benchmarks/hisparse_locality_replay.py:90-99 (misses counted at
 * entry, hits touched in selection order, least-recent evicted, misses
 * inserted in selection order). Replaces the policy part of the third-party
 * load_blocks_to_device_buffer_mha called at
 * adaptive_sparse/request_residency.py:805-809,829-832.
 *   topk [L, B, K] + block_size, rows [B], selected [S]: the lookup's inputs
 *   slots [L, B, W] int32: the lookup's output; miss lanes are patched in place
 *   misses [L, B, W], miss_count [L, B] int32: the lookup's miss list
 *   table [L, R, T] int32: token -> global slot (0 = not resident), or int16:
 *   token -> local slot + 1 (the form of ekv_resolve_resident_local), updated
 *   resident_bits [L, R, words] int32 or NULL: a residency summary of the
 *   table with bits_shift as in ekv_resolve_resident_bits; inserted tokens
 *   set their bit, and at bits_shift 0 evicted tokens clear theirs
 *   resident_counts NULL, or with resident_bits at bits_shift > 0:
 *   [L, R, ceil(T / 2^bits_shift)] int32, the resident positions under each
 *   summary bit (as the table holds them on entry), kept up to date; a bit
 *   is cleared when its count reaches zero, so the summary stays exact.
 *   Without them a coarse summary only gains bits and becomes a superset
 *   (ekv_residency_bits makes it exact again)
 *   slot_token [L, R, C] int32 (-1 = empty), stamps [L, R, C] int32: LRU state
 *   slot_base [R]: global slot of local slot 0 of each request's hot buffer
 *   (at least 1: global slot 0 is the sink that means "not resident", so a
 *   hot buffer starting there could never report its slot 0 as a hit)
 *   host_table [R, T]: token -> host row of the pinned host copy
 *   promote_src / promote_dst [L, B, W] int32: i < miss_count[l, b] get the
 *   host row and the global slot of the i-th promotion (feed to ekv_move_kv)
 *   status NULL or [1] int32 in device memory: EKV_SWAP_* bits are OR-ed in
 * Stamps are step * EKV_SWAP_STEP_STAMPS + lane (+ 4096 for a miss);
 * `step` must grow by one per call (the width W may change from call to
 * call) and keep (step + 1) * EKV_SWAP_STEP_STAMPS below 2^31, i.e.
 * step < 262143. W <= min(C, 4096), C <= 8192.
 * A token repeated within a row is one access by its first lane (the
 * replay's rule applied to the selection with later repeats dropped): its
 * later miss entries share the first one's slot and get empty promotions.
 * Selected rows naming the same request are refused (status
 * EKV_SWAP_SHARED_REQUEST). Miss-list entries that name no valid lane get
 * promote_src = promote_dst = -1, which ekv_move_kv skips. An empty batch
 * (B = 0) or selection launches nothing; a table without positions (T = 0)
 * is refused when there is work.
 */
int ekv_swap_in(const ekv_tensor* topk, int64_t block_size, const ekv_tensor* rows,
                const ekv_tensor* selected, const ekv_tensor* slots,
                const ekv_tensor* misses, const ekv_tensor* miss_count,
                const ekv_tensor* table, const ekv_tensor* resident_bits, int64_t bits_shift,
                const ekv_tensor* resident_counts, const ekv_tensor* slot_token, const ekv_tensor* stamps,
                const ekv_tensor* slot_base, const ekv_tensor* host_table,
                const ekv_tensor* promote_src, const ekv_tensor* promote_dst,
                int64_t step, const ekv_tensor* status, void* stream);

/*
 * ekv_swap_in with the step read from device memory: step_counter [1] int64
 * holds the step of this call and is incremented after the swap-in (a second
 * launch on the same stream), so a captured HIP graph replays consecutive
 * steps. The caller keeps (step + 1) * EKV_SWAP_STEP_STAMPS below 2^31 (rebasing the stamps
 * and the counter in time); a call past that limit changes nothing, records
 * empty promotions and sets EKV_SWAP_STAMP_OVERFLOW in `status`.
 * No reference counterpart: the graph-replayable form of ekv_swap_in.
 */
int ekv_swap_in_counted(const ekv_tensor* topk, int64_t block_size, const ekv_tensor* rows,
                        const ekv_tensor* selected, const ekv_tensor* slots,
                        const ekv_tensor* misses, const ekv_tensor* miss_count,
                        const ekv_tensor* table, const ekv_tensor* resident_bits, int64_t bits_shift,
                        const ekv_tensor* resident_counts, const ekv_tensor* slot_token,
                        const ekv_tensor* stamps, const ekv_tensor* slot_base, const ekv_tensor* host_table,
                        const ekv_tensor* promote_src, const ekv_tensor* promote_dst,
                        const ekv_tensor* step_counter, const ekv_tensor* status, void* stream);

/*
 * HiSparse hot-buffer swap-in with the calling convention of SGLang's
 * load_blocks_to_device_buffer_mha, which the reference's decode path calls
 * through its coordinator (adaptive_sparse/request_residency.py:805-809,
 * 829-832) and checks directly in tests/smoke_minimax_swap.py:38-67. For
 * batch row b < num_real_reqs[0] (NULL: every row), r = req_pool_indices[b],
 * s = seq_lens[b], H = hot_buffer_size:
 *   selected tokens: top_k_blocks[b, k] >= 0 expanded to block * bs + j
 *     (j < bs = sparse_block_size), kept when < s and < T, in Top-K order
 *     (adaptive_sparse/hisparse_access_trace.py:59-64);
 *   the newest token s - 1 -> device_buffer_locs[r, H] (reserved; not copied);
 *   a token held by slot i < H (device_buffer_tokens[r, i]) hits ->
 *     device_buffer_locs[r, i];
 *   misses take victims in batch-token LRU order (empty slots first, then
 *     the least recent in lru_slots[r]; benchmarks/hisparse_locality_replay.py
 *     :90-99), get their K and V rows copied from host row
 *     host_cache_locs[r, t] of `host_cache`, and enter device_buffer_tokens;
 *     lru_slots[r] becomes: unused empty slots, untouched slots (old order),
 *     hits, misses (selection order);
 *   top_k_device_locs[b] = device locations in selection order, then -1.
 * A token repeated in a row is classified by its first lane and shares its
 * location. Rows past num_real_reqs, with s <= 0 or with r outside the state
 * get -1 only and change nothing; misses whose host row lies outside the host
 * cache are left out; locations outside `device_buffer` are reported as -1.
 *   top_k_blocks [B, K] int32/int64; device_buffer_tokens [R, >= H+1] int32;
 *   host_cache_locs [R, T] and device_buffer_locs [R, >= H+1] int32/int64;
 *   lru_slots [R, H] int16/int32 (a permutation of 0..H-1);
 *   top_k_device_locs [B, K*bs] int32; req_pool_indices, seq_lens [B].
 *   host_cache / device_buffer: one layer of K and V planes (kv = 2), rows of
 *   item_size_bytes; host_cache addresses device-mapped pinned memory
 *   (ekv_host_device_pointer).
 * H <= 4096, K * bs <= min(H, 2048); the batch rows must name distinct
 * requests (one workgroup updates each request's state).
 */
int ekv_hisparse_swap_in(const ekv_tensor* top_k_blocks, const ekv_tensor* device_buffer_tokens,
                         const ekv_tensor* host_cache_locs, const ekv_tensor* device_buffer_locs,
                         const ekv_planes* host_cache, const ekv_planes* device_buffer,
                         const ekv_tensor* top_k_device_locs, const ekv_tensor* req_pool_indices,
                         const ekv_tensor* seq_lens, const ekv_tensor* lru_slots,
                         int64_t hot_buffer_size, int64_t sparse_block_size,
                         const ekv_tensor* num_real_reqs, void* stream);

/* Device address of pinned host memory (hipHostGetDevicePointer), for host
 * tensors pinned by their owner (e.g. torch's pin_memory). No reference
 * counterpart. */
int ekv_host_device_pointer(void* host, void** device);

/*
 * Row moves between two plane sets: for i < counts[l, b] and both kv planes,
 *   dst(l, kv)[dst_rows[l, b, i]] = src(l, kv)[src_rows[l, b, i]]
 * when 0 <= src row < src->rows and zero_below <= dst row < dst->rows (other
 * entries move nothing). src may be mapped pinned host memory
 * (ekv_host_alloc), which makes this the promote-from-host copy.
 * Replaces the byte movement of load_to_device_per_layer used by
 * adaptive_sparse/migration.py:232-237 for scattered token rows.
 */
int ekv_move_kv(const ekv_planes* src, const ekv_tensor* src_rows,
                const ekv_planes* dst, const ekv_tensor* dst_rows,
                const ekv_tensor* counts, int64_t zero_below, void* stream);

/*
 * Byte-exact comparison of K/V rows of two plane sets (same kv, row_bytes):
 *   equal[l, b, w] = 1 when, in every kv plane, row a_rows[l, b, w] of `a`
 *   equals row b_rows[l, b, w] of `b` byte for byte; 0 when a byte differs;
 *   -1 when either index lies outside [0, rows) of its planes (nothing read).
 *   a_rows, b_rows [L, B, W] int32/int64; equal [L, B, W] int32.
 * Replaces the int16 row comparisons of LogicalShadow.check / check_complete
 * (adaptive_sparse/logical_shadow.py:72-75, 108-123).
 */
int ekv_compare_kv(const ekv_planes* a, const ekv_tensor* a_rows, const ekv_planes* b,
                   const ekv_tensor* b_rows, const ekv_tensor* equal, void* stream);

/* The arguments of ekv_decode_step: those of the lookup, the swap-in, the
 * promote move and the gather it runs, with the intermediates left out. */
typedef struct ekv_step_args {
    const ekv_tensor* topk;           /* [L, B, K] Top-K block ids, -1 = padding */
    int64_t block_size;
    const ekv_tensor* rows;           /* [B] request of each batch row */
    const ekv_tensor* lengths;        /* [B] */
    const ekv_tensor* selected;       /* [S] batch rows to serve; they name distinct requests */
    const ekv_tensor* table;          /* [L, R, T]: int16 local slot + 1, or int32 global slot; 0 = not resident */
    const ekv_tensor* resident_bits;  /* NULL or its residency summary ... */
    int64_t bits_shift;               /* ... one bit per 2^bits_shift positions */
    const ekv_tensor* resident_counts; /* NULL or [L, R, groups] int32 resident positions per bit (shift > 0) */
    const ekv_tensor* slot_base;      /* [R] global slot of each request's local slot 0 */
    const ekv_tensor* slot_token;     /* [L, R, C] LRU state, as ekv_swap_in */
    const ekv_tensor* stamps;         /* [L, R, C] */
    int64_t step;                     /* the LRU step (>= 0), or -1 with step_counter */
    const ekv_tensor* step_counter;   /* NULL or [1] int64 in device memory (graph replays) */
    const ekv_tensor* status;         /* NULL or [1] int32: EKV_SWAP_* bits */
    const ekv_tensor* host_table;     /* [R, T] token -> row of the host planes */
    const ekv_planes* host;           /* K/V rows in mapped pinned host memory */
    const ekv_planes* pool;           /* the hot K/V pool */
    const ekv_tensor* slots;          /* out [L, B, K * block_size] int32: each lane's slot after the swap-in */
    const ekv_kv_rows* out;           /* out: the gathered K/V rows of every lane */
} ekv_step_args;

/*
 * Workspace bytes ekv_decode_step needs for L layers x B rows x W lanes per
 * row: the miss list and two promotion lists ([L, B, W] int32 each) and the
 * miss counts ([L, B] int32), each 256-byte aligned. UINT64_MAX on error.
 */
uint64_t ekv_decode_step_workspace_bytes(int64_t layers, int64_t batch, int64_t width);

/*
 * One decode step: ekv_resolve_resident_local (int16 table) /
 * ekv_resolve_resident_bits / ekv_resolve_resident with miss compaction ->
 * ekv_swap_in (or ekv_swap_in_counted with step_counter) -> ekv_move_kv of
 * the promotions from args->host into args->pool -> ekv_gather_kv of every
 * lane's slot into args->out, queued in that order on `stream`. Each stage
 * keeps its own entry point's contract; the miss list, counts and promotion
 * lists live in `workspace` (a 256-byte aligned device buffer of at least
 * ekv_decode_step_workspace_bytes; its contents on entry do not matter: the
 * counts are zeroed by a kernel first, so rows outside `selected` promote
 * nothing). After the step every selected lane's slot holds its token's row;
 * rows outside `selected` keep their slots and are gathered as they stand.
 * Records no memset, so the call can be captured in a HIP graph.
 * Replaces, for one layer or several: the lookup + host-backed swap of the
 * reference's decode path (adaptive_sparse/request_residency.py:805-832) and
 * the read of the selected rows that follows it.
 */
int ekv_decode_step(const ekv_step_args* args, void* workspace, uint64_t workspace_bytes, void* stream);

/*
 * ekv_decode_step without a workspace argument and without any allocation:
 * the miss list, counts and promotion lists live in a file-scope device
 * array of the library, 32 MiB per GPU (held from the first call until the
 * process ends), so the step may take at most
 * ekv_decode_step_workspace_bytes(L, B, W) <= 33554432 bytes (e.g. 8 layers
 * x 128 rows x 2048 lanes); a larger step fails with a message (split it over
 * fewer layers or rows). Every call on one GPU shares that array: calls that
 * overlap on one GPU (other streams, other threads) race, so they must be
 * ordered. Otherwise it behaves exactly as ekv_decode_step.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).
 */
int ekv_decode_step_static(const ekv_step_args* args, void* stream);

/* Modes of ekv_stream_probe. */
#define EKV_PROBE_READ 0   /* read src (fold, no stores)       */
#define EKV_PROBE_WRITE 1  /* write zeros to dst                */
#define EKV_PROBE_COPY 2   /* dst = src                         */
/* Variant flags, OR-ed into the mode. */
#define EKV_PROBE_NT_LOAD 0x10    /* non-temporal loads                       */
#define EKV_PROBE_HALF_TILE 0x20  /* 16 KiB tiles, 4 loads in flight per lane */

/*
 * Streaming bandwidth probe over `bytes` of dense device memory (16-byte
 * aligned, a multiple of 16): one launch of the read-only, write-only or
 * copy kernel, with the row-copy engine's access style (16-byte lanes, 8
 * loads in flight per lane, non-temporal stores, 32 KiB tiles dealt to the
 * XCDs in contiguous ranges); EKV_PROBE_NT_LOAD and EKV_PROBE_HALF_TILE
 * select the variants a ceiling is also taken over (the read and copy modes
 * take both, the write mode the tile size). workgroups_per_cu > 0 reserves LDS so that at
 * most that many workgroups share a CU; 0 leaves the register limit. dst must
 * hold `bytes` bytes in every mode (the read probe never writes it unless src
 * holds a planted pattern); src may be NULL for EKV_PROBE_WRITE.
 * No reference counterpart: the on-box ceilings the kernels above are
 * measured against.
 */
int ekv_stream_probe(int mode, const void* src, void* dst, uint64_t bytes, int workgroups_per_cu,
                     void* stream);

/* Pinned host memory (hipHostMalloc) plus the device pointer kernels use to
 * read and write it. Free with ekv_host_free(host). No reference counterpart
 * (the reference's pinned pools are SGLang's HostKVCache). */
int ekv_host_alloc(uint64_t bytes, void** host, void** device);
int ekv_host_free(void* host);

#ifdef __cplusplus
}
#endif

#endif /* EKV_KERNELS_H */
