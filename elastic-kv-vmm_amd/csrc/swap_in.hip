// Hot-buffer swap-in with batch-token LRU replacement (gfx950).
//
// Policy: benchmarks/hisparse_locality_replay.py:90-99 - per (request, layer)
// stream, misses are counted at entry, hits are touched (moved to most recent,
// in selection order), least-recent entries are evicted until the misses fit,
// then the misses are inserted in selection order. Here the hot buffer of a
// (layer, request) row is `capacity` slots; the reference's ordered dict is
// represented by one recency stamp per slot:
//   touched hit of lane o at step s: stamp = s * 8192 + o
//   inserted miss of lane o:         stamp = s * 8192 + 4096 + o
//   empty slot:                      stamp = INT32_MIN
// (a row has at most 4096 lanes, so every step's stamps lie above all of the
// steps before it whatever the width of each call), so sorting slots by
// (stamp, slot) reproduces the dict's order, and the m victims of a step
// (m = distinct missed tokens) are the slots of the m smallest keys: empty
// slots first, then the least recently used entries.
//
// Repeated tokens. The reference's replay refuses a selection that repeats a
// token (hisparse_locality_replay.py:55-56), but Top-K blocks expand to
// repeats when a block id appears twice (the access-trace KAT
// tests/test_hisparse_access_trace.py:170-199 selects [2, 3, 6, 2, 3]). This
// kernel defines a repeated token as one access by its first lane - the
// replay applied to the selection with later repeats dropped: a hit's stamp
// takes its lowest lane (atomicMin in LDS), a repeated miss takes one victim
// (an LDS hash of the miss tokens names each token's first miss), and its
// later lanes share that slot and record empty promotions.
//
// One 256-thread workgroup per (row, layer): hits are touched in LDS, a
// radix select over the stamps finds the victims (the slots of the smallest
// (stamp, slot) keys), which one scan lists in slot order; the i-th distinct
// miss (in miss-list order) takes the i-th of them. (Which victim slot a
// miss takes is this kernel's own convention: the reference's LRU is an
// ordered dict of tokens, whose contents and order do not depend on it.)
// Each victim clears its old token from the token->slot table and residency
// summary, takes the new token, and writes one promotion (host row -> global
// slot) record. The lookup's slot output of every miss lane is patched to its
// new slot, so the gather that follows reads the promoted row.
//
// Residency summary. At bits_shift 0 a bit is one position: an evicted
// token clears it, an inserted token sets it. A coarser bit covers 2^shift
// positions; with per-bit resident counts the summary stays exact: every
// eviction decrements its group's count and clears the bit when it reaches
// zero, then (after a workgroup barrier, so no clear can follow a set) every
// insertion increments its group's count and sets the bit from zero.
// Without counts a coarse bit is only ever set, and the summary is a
// superset of the table.
//
// Refused rows. Two selected rows naming one request would race on its hot
// buffer, and a step whose stamps would overflow int32 cannot be ordered:
// such a row changes nothing, records empty promotions and ORs
// EKV_SWAP_SHARED_REQUEST or EKV_SWAP_STAMP_OVERFLOW into the caller's
// status word, which the host reads back.
#include "../../include/ekv_kernels.h"
#include "ekv_common.h"
#include "ekv_fastdiv.h"
#include "ekv_tensor_util.h"

#include <algorithm>
#include <climits>

namespace ekv {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxCapacity = 8192;   // slots per hot buffer (stamps held in LDS; 16-bit scan fields)
constexpr int kMaxWidth = 4096;      // lanes per row whose miss tokens are hashed in LDS
static_assert(kMaxWidth <= 16 * kThreads && kMaxCapacity <= 32 * kThreads,
              "the kernel's register batches hold at most 16 lanes and 32 stamps per thread");
// Stamps per LRU step: hits take step * kStepStamps + lane, misses
// step * kStepStamps + kMaxWidth + lane, so a call with fewer lanes than the
// one before still stamps above it.
constexpr int64_t kStepStamps = EKV_SWAP_STEP_STAMPS;
static_assert(kStepStamps == 2 * kMaxWidth, "hit and miss stamps of one step take 2 * kMaxWidth values");
constexpr int32_t kStatusStampOverflow = EKV_SWAP_STAMP_OVERFLOW;
constexpr int32_t kStatusSharedRequest = EKV_SWAP_SHARED_REQUEST;

struct SwapArgs {
    const void* topk;
    int32_t topk64;
    int64_t topk_sl, topk_sb, topk_sk;
    uint32_t block_size;
    FastDiv block_div;
    IndexRef rows, selected, slot_base;
    int64_t selected_count;
    int32_t* slots;                 // [L, B, W] lookup output, patched for misses
    int64_t sl_l, sl_b, sl_o;
    const int32_t* misses;          // [L, B, W] miss lanes
    int64_t mi_l, mi_b, mi_o;
    const int32_t* counts;          // [L, B]
    int64_t ct_l, ct_b;
    void* table;                    // [L, R, T] token -> global slot (int32) or local slot + 1 (int16); 0 = not resident
    int32_t table16;
    int64_t tb_l, tb_r, tb_t, table_cols;
    int32_t* bits;                  // [L, R, words] residency summary (may be null)
    int64_t bt_l, bt_r, bt_w;
    uint32_t bits_shift;            // bit q covers positions [q << shift, (q + 1) << shift)
    int32_t* line_counts;           // [L, R, groups] resident positions per summary bit (bits_shift > 0; may be null)
    int64_t lc_l, lc_r, lc_q;
    int32_t* slot_token;            // [L, R, C] token held by each slot (-1 = empty)
    int64_t st_l, st_r, st_c;
    int32_t* stamps;                // [L, R, C] recency stamps
    int64_t sp_l, sp_r, sp_c;
    IndexRef host_table;            // [R, T] token -> host row, addressed with explicit strides
    int64_t host_sr, host_st;
    int32_t* promote_src;           // [L, B, W] host row per promotion
    int64_t ps_l, ps_b, ps_o;
    int32_t* promote_dst;           // [L, B, W] global slot per promotion
    int64_t pd_l, pd_b, pd_o;
    int64_t batch, table_rows, capacity;
    uint32_t width;
    int64_t step;
    const int64_t* step_counter;    // when set, the step is read from device memory (graph replays)
    int32_t* status;                // EKV_SWAP_* error bits, OR-ed in (may be null)
    uint32_t touched_words;         // ceil(C / 32): words of the touched-slot bits
    uint32_t hash_size, hash_log2;  // miss-token hash buckets: a power of two >= 2W (and >= 2)
    uint32_t token_bitmap;          // 1: T <= 16 * hash_size, the region first serves as a token bitmap
    uint32_t bitmap_words;          // ceil(T / 32)
};

// A Top-K id (int32 or int64 elements) without a branch on the element type:
// the low word, then the high word (for int32 ids the low word again,
// replaced by its sign). A branch per id would make the compiler wait for
// each load before issuing the next.
__device__ __forceinline__ int64_t load_id(const void* row, int32_t is64, int64_t index) {
    const char* at = static_cast<const char*>(row) + index * (is64 ? 8 : 4);
    const int32_t lo = *reinterpret_cast<const int32_t*>(at);
    const int32_t high = *reinterpret_cast<const int32_t*>(at + (is64 ? 4 : 0));
    return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(is64 ? high : lo >> 31)) << 32) |
                                static_cast<uint32_t>(lo));
}

// Writes a token -> slot table entry (int32 global slot or int16 local slot + 1).
__device__ __forceinline__ void set_entry(const SwapArgs& a, int64_t offset, int32_t value) {
    if (a.table16) {
        static_cast<int16_t*>(a.table)[offset] = static_cast<int16_t>(value);
    } else {
        static_cast<int32_t*>(a.table)[offset] = value;
    }
}

// Exclusive prefix sum of one int per thread over the workgroup (wave64
// shuffles, then one LDS exchange of the wave totals); `total` receives the
// sum. Every thread must call it.
__device__ __forceinline__ int32_t workgroup_exclusive_scan(int32_t value, int32_t* wave_totals, int32_t& total) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int32_t inclusive = value;
#pragma unroll
    for (int offset = 1; offset < 64; offset <<= 1) {
        const int32_t below = __shfl_up(inclusive, offset);
        inclusive += lane >= offset ? below : 0;
    }
    if (lane == 63) {
        wave_totals[wave] = inclusive;
    }
    __syncthreads();
    int32_t before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        before += w < wave ? wave_totals[w] : 0;
        total += wave_totals[w];
    }
    __syncthreads();  // wave_totals may be rewritten by the next scan
    return before + inclusive - value;
}

// A workgroup barrier that orders LDS only: waves wait for their own LDS
// accesses, not for their outstanding global stores (which a full
// __syncthreads would also wait for).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Lanes of this wave below the calling lane whose bit is set in `mask`.
__device__ __forceinline__ int32_t lanes_below(uint64_t mask) {
    return static_cast<int32_t>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                          __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}

// Sum, minimum and maximum of one value per thread over the workgroup
// (wave shuffles, then one LDS exchange of the wave results). Every thread
// must call it; `partial` holds 3 * (kThreads / 64) words.
__device__ __forceinline__ void workgroup_sum_min_max(uint32_t& sum, uint32_t& lo, uint32_t& hi, uint32_t* partial) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        sum += __shfl_xor(sum, offset);
        lo = min(lo, static_cast<uint32_t>(__shfl_xor(lo, offset)));
        hi = max(hi, static_cast<uint32_t>(__shfl_xor(hi, offset)));
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        partial[3 * wave] = sum;
        partial[3 * wave + 1] = lo;
        partial[3 * wave + 2] = hi;
    }
    lds_barrier();
    sum = 0;
    lo = 0xffffffffu;
    hi = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        sum += partial[3 * w];
        lo = min(lo, partial[3 * w + 1]);
        hi = max(hi, partial[3 * w + 2]);
    }
}

__device__ __forceinline__ uint32_t token_hash(int32_t token, uint32_t log2_size) {
    return (static_cast<uint32_t>(token) * 2654435761u) >> (32 - log2_size);
}

// Packed 16-bit buckets of the miss-token hash: bucket h is the half
// (h & 1) of word h >> 1; 0xffff marks an empty bucket, otherwise the bucket
// holds a miss index (< 4096).
constexpr uint32_t kEmptyBucket = 0xffffu;

__device__ __forceinline__ uint32_t bucket_of(const uint32_t* words, uint32_t h) {
    return (words[h >> 1] >> ((h & 1u) * 16u)) & 0xffffu;
}

// Writes `value` into bucket h when the bucket holds `expected`; the other
// half of the word is preserved (retried while another lane changes it).
// Returns the bucket's value before the write, or its current value when it
// no longer held `expected`.
__device__ __forceinline__ uint32_t bucket_cas(uint32_t* words, uint32_t h, uint32_t expected, uint32_t value) {
    const uint32_t shift = (h & 1u) * 16u;
    uint32_t* word = words + (h >> 1);
    uint32_t seen = *word;
    while (true) {
        const uint32_t held = (seen >> shift) & 0xffffu;
        if (held != expected) {
            return held;
        }
        const uint32_t desired = (seen & ~(0xffffu << shift)) | (value << shift);
        const uint32_t previous = atomicCAS(word, seen, desired);
        if (previous == seen) {
            return expected;
        }
        seen = previous;   // the word changed (this bucket or its neighbour): look again
    }
}

// Lowers bucket h to `value` when that is smaller (a 16-bit atomicMin).
__device__ __forceinline__ void bucket_min(uint32_t* words, uint32_t h, uint32_t value) {
    uint32_t held = bucket_of(words, h);
    while (value < held) {
        const uint32_t seen = bucket_cas(words, h, held, value);
        if (seen == held) {
            return;
        }
        held = seen;
    }
}

// Open-addressing hash of the miss tokens: every token ends up in one bucket
// holding its lowest miss index. The table holds at least 2m buckets, so
// every probe meets its token or an empty bucket. Every thread must call it.
__device__ __forceinline__ void hash_miss_tokens(uint32_t* hash, const int32_t* info, int32_t m, uint32_t log2_size) {
    const uint32_t mask = (1u << log2_size) - 1u;
    for (int32_t i = threadIdx.x; i < m; i += kThreads) {
        const int32_t token = info[i];
        if (token < 0) {
            continue;
        }
        uint32_t h = token_hash(token, log2_size);
        while (true) {
            const uint32_t held = bucket_cas(hash, h, kEmptyBucket, static_cast<uint32_t>(i));
            if (held == kEmptyBucket) {
                break;   // claimed
            }
            if (info[held] == token) {
                bucket_min(hash, h, static_cast<uint32_t>(i));
                break;
            }
            h = (h + 1) & mask;
        }
    }
}

// Dynamic LDS of one workgroup (C = capacity, W = lanes per row):
//   stamp    int32 [C]  recency stamps;
//   info     int32 [W]  token of miss i (-1: an entry naming no valid lane);
//   touched  uint32 [ceil(C / 32)]  one bit per slot a hit touches;
//   region   hash_size 16-bit buckets (the miss-token hash), then the int16
//            list of the victims' slots in slot order;
//   owner    int16 [W]  the first miss of the same token (-1: an entry naming
//            no valid lane); a first miss's own entry then becomes -2 - the
//            rank of its victim.
// 36.5 KiB at C = 4096, W = 2048, so 4 workgroups share a CU.
//
// Global reads come in three batches, each issued as a fixed number of
// unrolled loads from clamped, in-bounds addresses and waited for once: the
// stamps, lookup slots and miss list (with the request checks); the Top-K
// ids of the miss entries; the victims' old tokens and host rows. (A loop
// with a run-time trip count waits for each load before issuing the next: a
// workgroup then spends most of its life on a chain of HBM round trips.)
// kSlotRegs >= C / kThreads stamps and kLaneRegs >= W / kThreads lanes per
// thread are held in registers.
template <int kSlotRegs, int kLaneRegs>
__global__ __launch_bounds__(kThreads) void swap_in_kernel(const SwapArgs a) {
    extern __shared__ __align__(16) unsigned char shared[];
    __shared__ int32_t wave_totals[kThreads / 64];
    __shared__ int32_t digit_count[2][256];   // radix-select histograms of one 8-bit digit (two passes)
    __shared__ int32_t chosen[2];          // the digit holding the need-th key, and the keys below it
    __shared__ uint32_t key_range[3 * (kThreads / 64)];   // empties, smallest and largest other key per wave
    __shared__ int32_t row_counts[2][kSlotRegs][kThreads / 64];   // keys below T / at T per (row, wave)
    int32_t* stamp = reinterpret_cast<int32_t*>(shared);
    int32_t* info = stamp + a.capacity;
    uint32_t* touched = reinterpret_cast<uint32_t*>(info + a.width);
    uint32_t* hash = touched + a.touched_words;
    int16_t* victims = reinterpret_cast<int16_t*>(hash);
    int16_t* owner = reinterpret_cast<int16_t*>(hash + a.hash_size / 2);
    // The prologue's reads are vector loads issued together: as scalar loads
    // (uniform reads) the compiler waited for each before the next one, and
    // the selection entry, request row, miss count, step and slot base were a
    // chain of round trips. The request row and miss count are read on the
    // guess that the selection is the identity (entry j names batch row j:
    // every batch row, the decode default); a different entry re-reads them
    // for its row. The slot base is read beside batch 1, with whose results
    // it is first needed.
    const uint32_t zero = opaque_zero();
    const int64_t l = blockIdx.y;
    const int64_t guess = blockIdx.x < a.batch ? blockIdx.x : 0;
    const PendingIndex entry_read = issue_index(a.selected, blockIdx.x, zero);
    const PendingIndex req_read = issue_index(a.rows, guess, zero);
    const int32_t counted_read = a.counts[l * a.ct_l + guess * a.ct_b + zero];
    // The device step of a graph replay; without one, a word of the counts
    // stands in and is not used.
    const bool device_step = a.step_counter != nullptr;   // uniform
    const int32_t* step_words = device_step ? reinterpret_cast<const int32_t*>(a.step_counter) : a.counts;
    const int32_t step_lo = step_words[zero];
    const int32_t step_hi = step_words[(device_step ? 1u : 0u) + zero];
    // Every value is read back before the first early return, so the loads
    // stay together (the compiler moves a load whose uses all lie past a
    // return below it, where it waits for it alone).
    const int64_t b = index_value(a.selected, entry_read);
    int64_t req = index_value(a.rows, req_read);
    int32_t counted = __builtin_amdgcn_readfirstlane(counted_read);
    const int64_t step =
        device_step ? static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(
                                                __builtin_amdgcn_readfirstlane(step_hi))) << 32) |
                                           static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(step_lo)))
                    : a.step;   // uniform
    const bool live = b >= 0 && b < a.batch;   // uniform
    if (live && b != guess) {   // uniform: the selection is not the identity here
        req = a.rows.fetch(b);
        counted = a.counts[l * a.ct_l + b * a.ct_b];
    }
    if (!live || req < 0 || req >= a.table_rows) {
        return;  // uniform: a stray selection, or a row outside the tables (nothing resident)
    }
    const int64_t C = a.capacity;
    const int64_t W = a.width;
    const PendingIndex base_read = issue_index(a.slot_base, req, zero);
    int32_t* promote_src = a.promote_src + l * a.ps_l + b * a.ps_b;
    int32_t* promote_dst = a.promote_dst + l * a.pd_l + b * a.pd_b;
    int32_t* slots = a.slots + l * a.sl_l + b * a.sl_b;
    const int64_t table_row = l * a.tb_l + req * a.tb_r;   // element offset of this (layer, request) row
    int32_t* slot_token = a.slot_token + l * a.st_l + req * a.st_r;
    int32_t* stamps = a.stamps + l * a.sp_l + req * a.sp_r;
    const int32_t* misses = a.misses + l * a.mi_l + b * a.mi_b;
    const void* topk_row = a.topk64
        ? static_cast<const void*>(static_cast<const int64_t*>(a.topk) + l * a.topk_sl + b * a.topk_sb)
        : static_cast<const void*>(static_cast<const int32_t*>(a.topk) + l * a.topk_sl + b * a.topk_sb);

    // One workgroup owns each (layer, request) hot buffer: a second selected
    // row naming the same request would race on it, so both rows are refused.
    // Thread t checks selection entry t (and t + kThreads, ... for longer
    // selections). Vector loads complete in issue order, so entry t is read
    // before batch 1 and its request row right after batch 1 is issued: batch 2
    // then waits for batch 1 alone, not for two dependent reads behind it.
    const int64_t selected_count = a.selected_count;   // at least 1
    const int64_t first_j = threadIdx.x;
    const int64_t first_other = a.selected.fetch(first_j < selected_count ? first_j : selected_count - 1);
    // Batch 1: stamps, the lookup slots of this thread's lanes, its miss-list entries.
    int32_t held_stamp[kSlotRegs];
#pragma unroll
    for (int k = 0; k < kSlotRegs; ++k) {
        const int64_t s = min(static_cast<int64_t>(threadIdx.x) + int64_t{k} * kThreads, C - 1);
        held_stamp[k] = stamps[s * a.sp_c];
    }
    int32_t lane_slot[kLaneRegs];
    int32_t miss_lane[kLaneRegs];
#pragma unroll
    for (int k = 0; k < kLaneRegs; ++k) {
        const int64_t o = min(static_cast<int64_t>(threadIdx.x) + int64_t{k} * kThreads, W - 1);
        lane_slot[k] = slots[o * a.sl_o];
        miss_lane[k] = misses[o * a.mi_o];   // entries at or past the count are read but not used
    }
    const bool first_in_range =
        first_j < selected_count && first_j != blockIdx.x && first_other >= 0 && first_other < a.batch;
    const int64_t first_req = a.rows.fetch(first_in_range ? first_other : b);   // b is a valid batch row
    bool shared_request = first_in_range && first_req == req;
    for (int64_t j = first_j + kThreads; j < selected_count; j += kThreads) {
        const int64_t other = a.selected[j];
        shared_request |= j != blockIdx.x && other >= 0 && other < a.batch && a.rows[other] == req;
    }
    // Batch 2: the Top-K ids of the miss entries.
    int64_t miss_block[kLaneRegs];
#pragma unroll
    for (int k = 0; k < kLaneRegs; ++k) {
        const uint32_t lane = static_cast<uint32_t>(min(max(miss_lane[k], 0), static_cast<int32_t>(W - 1)));
        const uint32_t blk = a.block_size == 1 ? lane : a.block_div.div(lane);
        miss_block[k] = load_id(topk_row, a.topk64, blk * a.topk_sk);
    }
    const int32_t m = counted < 0 ? 0 : (counted > W ? static_cast<int32_t>(W) : counted);
    shared_request = __syncthreads_or(shared_request);
    const bool overflow = step < 0 || (step + 1) * kStepStamps >= (int64_t{1} << 31);
    if (shared_request || overflow) {
        // Change nothing, record empty promotions (the move that follows
        // copies nothing; the missed lanes keep slot 0) and flag the error.
        if (threadIdx.x == 0 && a.status != nullptr) {
            atomicOr(a.status, shared_request ? kStatusSharedRequest : kStatusStampOverflow);
        }
        for (int64_t i = threadIdx.x; i < m; i += kThreads) {
            promote_src[i * a.ps_o] = -1;
            promote_dst[i * a.pd_o] = -1;
        }
        return;
    }
    const int64_t stamp_base = step * kStepStamps;
#pragma unroll
    for (int k = 0; k < kSlotRegs; ++k) {
        const int64_t s = threadIdx.x + int64_t{k} * kThreads;
        if (s < C) {
            stamp[s] = held_stamp[k];
        }
    }
    const int64_t base = index_value(a.slot_base, base_read);
    int32_t hit_local[kLaneRegs];   // local slot a lane hits, or -1
#pragma unroll
    for (int k = 0; k < kLaneRegs; ++k) {
        const int64_t o = threadIdx.x + int64_t{k} * kThreads;
        const int64_t offset = static_cast<int64_t>(lane_slot[k]) - base;
        hit_local[k] = o < W && lane_slot[k] > 0 && offset >= 0 && offset < C ? static_cast<int32_t>(offset) : -1;
        const int64_t i = o;   // this thread's k-th miss-list entry
        if (i < m) {
            const int32_t lane = miss_lane[k];
            const int64_t offset_in_block =
                a.block_size == 1 ? 0 : static_cast<int64_t>(lane) - int64_t{a.block_div.div(static_cast<uint32_t>(lane))} *
                                                                          a.block_size;
            const int64_t token = lane >= 0 && lane < W ? miss_block[k] * a.block_size + offset_in_block : int64_t{-1};
            info[i] = token >= 0 && token < a.table_cols ? static_cast<int32_t>(token) : -1;
        }
    }
    for (uint32_t w = threadIdx.x; w < a.touched_words; w += kThreads) {
        touched[w] = 0;
    }
    // The region starts as a token bitmap (all clear) when the tokens fit it,
    // else as the empty hash.
    const uint32_t region_words = a.token_bitmap ? a.bitmap_words : a.hash_size / 2;
    const uint32_t region_fill = a.token_bitmap ? 0u : 0xffffffffu;
    for (uint32_t w = threadIdx.x; w < region_words; w += kThreads) {
        hash[w] = region_fill;
    }
    __syncthreads();
    // Touch hits. A token repeated in the row is one access of its first lane:
    // a touched slot's stamp becomes stamp_base + the lowest lane that hit it
    // (marked, raised to INT32_MAX, then lowered by every hitting lane).
#pragma unroll
    for (int k = 0; k < kLaneRegs; ++k) {
        if (hit_local[k] >= 0) {
            atomicOr(&touched[hit_local[k] >> 5], 1u << (hit_local[k] & 31));
        }
    }
    // Repeated miss tokens. With the token bitmap, each valid entry sets its
    // token's bit; a bit found set means some token repeats, and only then is
    // the exact hash built (each token's lowest miss index). Without repeats
    // every valid entry is its token's first miss.
    bool repeated = false;
    if (a.token_bitmap) {   // uniform
#pragma unroll
        for (int k = 0; k < kLaneRegs; ++k) {
            const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kThreads;
            const int32_t token = i < m ? info[i] : -1;
            if (token >= 0) {
                const uint32_t bit = 1u << (token & 31);
                repeated |= (atomicOr(&hash[token >> 5], bit) & bit) != 0u;
            }
        }
    } else {
        hash_miss_tokens(hash, info, m, a.hash_log2);
    }
    const bool exact_hash = !a.token_bitmap || __syncthreads_or(repeated);   // uniform
    if (a.token_bitmap && exact_hash) {
        for (uint32_t w = threadIdx.x; w < a.hash_size / 2; w += kThreads) {
            hash[w] = 0xffffffffu;
        }
        __syncthreads();
        hash_miss_tokens(hash, info, m, a.hash_log2);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kSlotRegs; ++k) {
        const uint32_t s = threadIdx.x + k * kThreads;
        if (s < C && ((touched[s >> 5] >> (s & 31)) & 1u)) {
            stamp[s] = INT32_MAX;
        }
    }
    const uint32_t mask = a.hash_size - 1;
#pragma unroll
    for (int k = 0; k < kLaneRegs; ++k) {
        const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kThreads;
        if (i >= m) {
            continue;
        }
        const int32_t token = info[i];
        int32_t first = -1;
        if (token >= 0 && !exact_hash) {
            first = i;
        } else if (token >= 0) {
            for (uint32_t h = token_hash(token, a.hash_log2);; h = (h + 1) & mask) {
                const uint32_t held = bucket_of(hash, h);
                if (held == kEmptyBucket) {
                    break;   // not reached: every inserted token lies on its probe path
                }
                if (info[held] == token) {
                    first = static_cast<int32_t>(held);
                    break;
                }
            }
        }
        owner[i] = static_cast<int16_t>(first);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kLaneRegs; ++k) {
        if (hit_local[k] >= 0) {
            atomicMin(&stamp[hit_local[k]],
                      static_cast<int32_t>(stamp_base + threadIdx.x + static_cast<int64_t>(k) * kThreads));
        }
    }
    if (m > 0) {
        // Rank of each first miss among the first misses, in miss-list order:
        // every thread counts a contiguous run of entries, one scan. (The
        // scan's barriers also order the touches above before the select.)
        const int32_t per_thread = (m + kThreads - 1) / kThreads;
        const int32_t run_begin = min(m, static_cast<int32_t>(threadIdx.x) * per_thread);
        const int32_t run_end = min(m, run_begin + per_thread);
        int32_t firsts = 0;
        for (int32_t i = run_begin; i < run_end; ++i) {
            firsts += owner[i] == i;
        }
        int32_t unique = 0;
        int32_t rank = workgroup_exclusive_scan(firsts, wave_totals, unique);
        for (int32_t i = run_begin; i < run_end; ++i) {
            if (owner[i] == i) {
                owner[i] = static_cast<int16_t>(-2 - rank++);   // a first miss: its victim's rank, below -1
            }
        }
        // The `unique` victims: the slots of the smallest (stamp, slot) keys,
        // empty slots (INT32_MIN) first, then the least recently used. In
        // the order-preserving unsigned form of the stamps an empty slot is
        // key 0. When the empties do not cover the victims, a radix select
        // over the other keys (8-bit digits, most significant first) finds
        // the key T of the (unique - empties)-th smallest of them and how
        // many keys at T it takes; it starts at the highest digit where the
        // smallest and largest of those keys differ (the stamps of a buffer
        // span a few steps: two digits). The victims are then listed in slot
        // order, and the i-th first miss takes the i-th of them.
        if (unique > 0) {   // uniform
            // This thread's keys, slots t + 256 k, read once (the touches
            // landed before the rank scan's barriers); 0xffffffff past C.
            uint32_t key[kSlotRegs];
#pragma unroll
            for (int k = 0; k < kSlotRegs; ++k) {
                const uint32_t s = threadIdx.x + k * kThreads;
                key[k] = s < C ? static_cast<uint32_t>(stamp[s]) ^ 0x80000000u : 0xffffffffu;
            }
            digit_count[0][threadIdx.x] = 0;   // the first pass's histogram; the reduction's barrier follows
            uint32_t empties = 0, lo = 0xffffffffu, hi = 0;
#pragma unroll
            for (int k = 0; k < kSlotRegs; ++k) {
                const uint32_t v = key[k];
                const bool other = v != 0 && threadIdx.x + k * kThreads < C;
                empties += v == 0 ? 1u : 0u;
                lo = other ? min(lo, v) : lo;
                hi = other ? max(hi, v) : hi;
            }
            workgroup_sum_min_max(empties, lo, hi, key_range);
            uint32_t prefix = 0, prefix_mask = 0xffffffffu;
            int32_t need = unique;   // keys still to take at the prefix (uniform)
            int first_shift = -8;    // no select: the empties alone, or every other key equal
            if (static_cast<uint32_t>(unique) > empties) {
                need = unique - static_cast<int32_t>(empties);
                const uint32_t differ = lo ^ hi;
                prefix = lo;
                if (differ != 0) {
                    first_shift = ((31 - __clz(differ)) / 8) * 8;
                    prefix_mask = first_shift == 24 ? 0u : ~((1u << (first_shift + 8)) - 1u);
                    prefix = lo & prefix_mask;
                }
            }
            for (int shift = first_shift, pass = 0; shift >= 0; shift -= 8, ++pass) {
                int32_t* count = digit_count[pass & 1];
                // Runs of one digit in a thread's slots count with one atomic:
                // recent stamps share their high digits, which would otherwise
                // serialize thousands of atomics on one counter.
                uint32_t run_digit = 0;
                int32_t run = 0;
#pragma unroll
                for (int k = 0; k < kSlotRegs; ++k) {
                    const uint32_t v = key[k];
                    if (v != 0 && (v & prefix_mask) == prefix && threadIdx.x + k * kThreads < C) {
                        const uint32_t d = (v >> shift) & 255u;
                        if (run > 0 && d != run_digit) {
                            atomicAdd(&count[run_digit], run);
                            run = 0;
                        }
                        run_digit = d;
                        ++run;
                    }
                }
                if (run > 0) {
                    atomicAdd(&count[run_digit], run);
                }
                lds_barrier();
                // Wave 0 scans the 256 counts (4 digits per lane) and names the
                // digit holding the need-th key; the others clear the next
                // pass's histogram meanwhile.
                if (threadIdx.x < 64) {
                    int32_t c[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        c[j] = count[4 * threadIdx.x + j];
                    }
                    const int32_t mine = c[0] + c[1] + c[2] + c[3];
                    int32_t inclusive = mine;
#pragma unroll
                    for (int offset = 1; offset < 64; offset <<= 1) {
                        const int32_t lower = __shfl_up(inclusive, offset);
                        inclusive += threadIdx.x >= static_cast<uint32_t>(offset) ? lower : 0;
                    }
                    int32_t below = inclusive - mine;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (below < need && need <= below + c[j]) {   // exactly one digit holds the need-th key
                            chosen[0] = static_cast<int32_t>(4 * threadIdx.x + j);
                            chosen[1] = below;
                        }
                        below += c[j];
                    }
                }
                for (uint32_t d = threadIdx.x; d < 256; d += kThreads) {
                    digit_count[(pass + 1) & 1][d] = 0;
                }
                lds_barrier();
                prefix |= static_cast<uint32_t>(chosen[0]) << shift;
                prefix_mask |= 255u << shift;
                need -= chosen[1];
            }
            // T = prefix. Slot s is a victim when its key is below T (every
            // empty slot, when the empties do not cover the victims), or at T
            // and fewer than `need` slots below s hold T; its place in the list
            // is the number of victims below it. Thread t takes slots
            // t + 256 k (conflict-free LDS reads); the slot-order counts of
            // both kinds come from per-wave ballots over each row of 256 slots.
            const int wave = threadIdx.x >> 6;
            uint32_t my_lower = 0, my_tie = 0;
#pragma unroll
            for (int k = 0; k < kSlotRegs; ++k) {
                const uint32_t s = threadIdx.x + k * kThreads;
                const uint32_t v = key[k];
                const bool lower = s < C && v < prefix;
                const bool tie = s < C && v == prefix;
                const uint64_t lower_lanes = __ballot(lower);
                const uint64_t tie_lanes = __ballot(tie);
                my_lower |= lower ? 1u << k : 0u;
                my_tie |= tie ? 1u << k : 0u;
                if ((threadIdx.x & 63) == 0) {
                    row_counts[0][k][wave] = __popcll(lower_lanes);
                    row_counts[1][k][wave] = __popcll(tie_lanes);
                }
            }
            lds_barrier();
            // Lane j < kSlotRegs of each wave takes row j: its keys of each kind
            // in all waves and in the waves below this one; a shuffle scan over
            // the lanes adds the rows below j, and the row loop reads row k's
            // base from lane k.
            const int lane = threadIdx.x & 63;
            int32_t row_lower = 0, row_tie = 0, wave_lower = 0, wave_tie = 0;
            if (lane < kSlotRegs) {
#pragma unroll
                for (int w = 0; w < kThreads / 64; ++w) {
                    const int32_t lower_here = row_counts[0][lane][w];
                    const int32_t tie_here = row_counts[1][lane][w];
                    row_lower += lower_here;
                    row_tie += tie_here;
                    wave_lower += w < wave ? lower_here : 0;
                    wave_tie += w < wave ? tie_here : 0;
                }
            }
            int32_t lower_scan = row_lower, tie_scan = row_tie;
#pragma unroll
            for (int offset = 1; offset < kSlotRegs; offset <<= 1) {
                const int32_t lower_up = __shfl_up(lower_scan, offset);
                const int32_t tie_up = __shfl_up(tie_scan, offset);
                lower_scan += lane >= offset ? lower_up : 0;
                tie_scan += lane >= offset ? tie_up : 0;
            }
            const int32_t lower_base = lower_scan - row_lower + wave_lower;   // row `lane`'s base for this wave
            const int32_t tie_base = tie_scan - row_tie + wave_tie;
#pragma unroll
            for (int k = 0; k < kSlotRegs; ++k) {
                const bool lower = (my_lower >> k) & 1u;
                const bool tie = (my_tie >> k) & 1u;
                const int32_t lower_before = __builtin_amdgcn_readlane(lower_base, k) + lanes_below(__ballot(lower));
                const int32_t ties_before = __builtin_amdgcn_readlane(tie_base, k) + lanes_below(__ballot(tie));
                if (lower || (tie && ties_before < need)) {
                    victims[lower_before + min(ties_before, need)] = static_cast<int16_t>(threadIdx.x + k * kThreads);
                }
            }
            lds_barrier();
        }
        int32_t* bits = a.bits != nullptr ? a.bits + l * a.bt_l + req * a.bt_r : nullptr;
        // Group counts keep a coarse summary exact: decrements here, increments after the barrier.
        int32_t* line_counts = bits != nullptr && a.bits_shift > 0 && a.line_counts != nullptr
                                   ? a.line_counts + l * a.lc_l + req * a.lc_r
                                   : nullptr;
        // Batch 3: each entry's victim (from LDS), then the victims' old
        // tokens and the promoted tokens' host rows, all loads issued before
        // any is used. Entry encoding: -1 names no valid lane; <= -2 is a
        // first miss, whose victim has rank -2 - entry; otherwise the index
        // of its first miss.
        int32_t entry_of[kLaneRegs];
        int32_t victim_of[kLaneRegs];
        int32_t old_of[kLaneRegs];
        int32_t host_row_of[kLaneRegs];
#pragma unroll
        for (int k = 0; k < kLaneRegs; ++k) {
            const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kThreads;
            const int32_t entry = i < m ? static_cast<int32_t>(owner[i]) : -1;
            const int32_t rank = entry == -1 ? 0 : -2 - (entry <= -2 ? entry : static_cast<int32_t>(owner[entry]));
            const int32_t victim = entry == -1 ? 0 : static_cast<int32_t>(static_cast<uint16_t>(victims[rank]));
            const int64_t token = entry == -1 ? 0 : info[i];   // >= 0 for an entry with a valid lane
            entry_of[k] = entry;
            victim_of[k] = victim;
            old_of[k] = slot_token[static_cast<int64_t>(victim) * a.st_c];
            host_row_of[k] = a.host_table.low(req * a.host_sr + token * a.host_st);
        }
#pragma unroll
        for (int k = 0; k < kLaneRegs; ++k) {
            const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kThreads;
            if (i >= m) {
                continue;
            }
            const int32_t entry = entry_of[k];
            const int32_t lane = miss_lane[k];
            if (entry == -1) {
                // Not an entry of a miss list written by the lookup: record an
                // empty promotion so the move that follows skips it.
                promote_src[i * a.ps_o] = -1;
                promote_dst[i * a.pd_o] = -1;
                continue;
            }
            const bool first = entry <= -2;
            const int64_t victim = victim_of[k];
            const int32_t global = static_cast<int32_t>(base + victim);
            const int64_t token = info[i];
            const int32_t old = old_of[k];
            const int32_t host_row = host_row_of[k];
            slots[static_cast<int64_t>(lane) * a.sl_o] = global;
            if (!first) {
                // A repeat of an earlier miss: it shares that miss's slot and promotion.
                promote_src[i * a.ps_o] = -1;
                promote_dst[i * a.pd_o] = -1;
                continue;
            }
            if (old >= 0 && old < a.table_cols) {
                set_entry(a, table_row + old * a.tb_t, 0);
                if (bits != nullptr && a.bits_shift == 0) {
                    atomicAnd(reinterpret_cast<unsigned int*>(bits + (old >> 5) * a.bt_w), ~(1u << (old & 31)));
                } else if (line_counts != nullptr) {
                    // The group's last resident position leaves: clear its bit.
                    const int64_t q = old >> a.bits_shift;
                    if (atomicSub(line_counts + q * a.lc_q, 1) == 1) {
                        atomicAnd(reinterpret_cast<unsigned int*>(bits + (q >> 5) * a.bt_w), ~(1u << (q & 31)));
                    }
                }
                // Without counts a coarse bit stays set (other positions of
                // its group may still be resident): a superset.
            }
            set_entry(a, table_row + token * a.tb_t, a.table16 ? static_cast<int32_t>(victim + 1) : global);
            if (bits != nullptr && line_counts == nullptr) {
                const int64_t q = token >> a.bits_shift;
                atomicOr(reinterpret_cast<unsigned int*>(bits + (q >> 5) * a.bt_w), 1u << (q & 31));
            }
            slot_token[victim * a.st_c] = static_cast<int32_t>(token);
            stamp[victim] = static_cast<int32_t>(stamp_base + kMaxWidth + lane);
            promote_src[i * a.ps_o] = host_row;
            promote_dst[i * a.pd_o] = global;
        }
        if (line_counts != nullptr) {   // uniform
            __syncthreads();   // the evictions' count decrements (global atomics) precede the increments
            // Insertions: after every eviction's clear above, so a group that
            // both loses and gains positions ends with its bit set.
            for (int32_t i = threadIdx.x; i < m; i += kThreads) {
                if (owner[i] <= -2) {   // a first miss: info[i] is its valid token
                    const int64_t q = static_cast<int64_t>(info[i]) >> a.bits_shift;
                    if (atomicAdd(line_counts + q * a.lc_q, 1) == 0) {
                        atomicOr(reinterpret_cast<unsigned int*>(bits + (q >> 5) * a.bt_w), 1u << (q & 31));
                    }
                }
            }
        } else {
            lds_barrier();     // the victims' stamps land in LDS before the write-back
        }
    } else {
        __syncthreads();   // the touches above land before the stamps are written back
    }
    for (int64_t s = threadIdx.x; s < C; s += kThreads) {
        stamps[s * a.sp_c] = stamp[s];
    }
}

// One thread advances the device step counter after the swap-in of a replay.
__global__ void advance_step_kernel(int64_t* counter) {
    if (threadIdx.x == 0) {
        counter[0] += 1;
    }
}

void need_i32(const ekv_tensor& t, const char* name) {
    if (t.dtype != EKV_INT32) {
        throw std::invalid_argument(std::string(name) + " must be int32");
    }
}

int swap_in(const ekv_tensor* topk_p, int64_t block_size, const ekv_tensor* rows_p, const ekv_tensor* selected_p,
            const ekv_tensor* slots_p, const ekv_tensor* misses_p, const ekv_tensor* counts_p,
            const ekv_tensor* table_p, const ekv_tensor* bits_p, int64_t bits_shift, const ekv_tensor* counts_q_p,
            const ekv_tensor* slot_token_p,
            const ekv_tensor* stamps_p, const ekv_tensor* slot_base_p, const ekv_tensor* host_table_p,
            const ekv_tensor* promote_src_p, const ekv_tensor* promote_dst_p, int64_t step,
            const ekv_tensor* step_counter_p, const ekv_tensor* status_p, void* stream) {
    const ekv_tensor& topk = need(topk_p, "topk");
    const ekv_tensor& rows = need(rows_p, "rows");
    const ekv_tensor& selected = need(selected_p, "selected");
    const ekv_tensor& slots = need(slots_p, "slots");
    const ekv_tensor& misses = need(misses_p, "misses");
    const ekv_tensor& counts = need(counts_p, "miss_count");
    const ekv_tensor& table = need(table_p, "table");
    const ekv_tensor& slot_token = need(slot_token_p, "slot_token");
    const ekv_tensor& stamps = need(stamps_p, "stamps");
    const ekv_tensor& slot_base = need(slot_base_p, "slot_base");
    const ekv_tensor& host_table = need(host_table_p, "host_table");
    const ekv_tensor& promote_src = need(promote_src_p, "promote_src");
    const ekv_tensor& promote_dst = need(promote_dst_p, "promote_dst");
    need_ndim(topk, 3, "topk");
    need_index(topk, "topk");
    const int64_t L = topk.shape[0], B = topk.shape[1], K = topk.shape[2];
    if (block_size < 1 || block_size >= (int64_t{1} << 31)) {
        throw std::invalid_argument("block_size must be positive");
    }
    const int64_t W = K * block_size;
    for (const auto* t : {&slots, &misses, &promote_src, &promote_dst}) {
        need_ndim(*t, 3, "slots/misses/promote lists");
        need_i32(*t, "slots/misses/promote lists");
        need_dim(*t, 0, L, "slots/misses/promote lists");
        need_dim(*t, 1, B, "slots/misses/promote lists");
        need_dim(*t, 2, W, "slots/misses/promote lists");
    }
    need_ndim(counts, 2, "miss_count");
    need_i32(counts, "miss_count");
    need_dim(counts, 0, L, "miss_count");
    need_dim(counts, 1, B, "miss_count");
    for (const auto* t : {&table, &slot_token, &stamps}) {
        need_ndim(*t, 3, "table/slot_token/stamps");
        if (t != &table || table.dtype != EKV_INT16) {
            need_i32(*t, "table/slot_token/stamps");
        }
        need_dim(*t, 0, L, "table/slot_token/stamps");
    }
    const int64_t R = table.shape[1], T = table.shape[2], C = slot_token.shape[2];
    need_dim(slot_token, 1, R, "slot_token");
    need_dim(stamps, 1, R, "stamps");
    need_dim(stamps, 2, C, "stamps");
    if (C < 1 || C > kMaxCapacity) {
        throw std::invalid_argument("capacity must be 1.." + std::to_string(kMaxCapacity));
    }
    static_assert(kMaxCapacity < 32768, "int16 tables hold local slot + 1");
    if (W > C) {
        throw std::invalid_argument("lanes per row exceed the hot capacity");
    }
    if (W > kMaxWidth) {
        throw std::invalid_argument("at most " + std::to_string(kMaxWidth) + " lanes per row");
    }
    if (T >= (int64_t{1} << 31) || step < 0 || (step + 1) * kStepStamps >= (int64_t{1} << 31)) {
        throw std::invalid_argument("token count or step outside the 32-bit stamp range");
    }
    int32_t* status = nullptr;
    if (status_p != nullptr) {
        const ekv_tensor& st = need(status_p, "status");
        if (st.dtype != EKV_INT32 || numel(st) != 1 || st.data == nullptr) {
            throw std::invalid_argument("status must be one int32 element in device memory");
        }
        status = static_cast<int32_t*>(st.data);
    }
    int64_t* counter = nullptr;
    if (step_counter_p != nullptr) {
        const ekv_tensor& c = need(step_counter_p, "step_counter");
        if (c.dtype != EKV_INT64 || numel(c) != 1 || c.data == nullptr) {
            throw std::invalid_argument("step_counter must be one int64 element in device memory");
        }
        counter = static_cast<int64_t*>(c.data);
    }
    need_ndim(rows, 1, "rows");
    need_ndim(selected, 1, "selected");
    need_ndim(slot_base, 1, "slot_base");
    need_index(rows, "rows");
    need_index(selected, "selected");
    need_index(slot_base, "slot_base");
    need_dim(rows, 0, B, "rows");
    need_dim(slot_base, 0, R, "slot_base");
    need_ndim(host_table, 2, "host_table");
    need_index(host_table, "host_table");
    need_dim(host_table, 0, R, "host_table");
    need_dim(host_table, 1, T, "host_table");
    if (bits_p != nullptr) {
        const ekv_tensor& bits = need(bits_p, "resident_bits");
        need_ndim(bits, 3, "resident_bits");
        need_i32(bits, "resident_bits");
        need_dim(bits, 0, L, "resident_bits");
        need_dim(bits, 1, R, "resident_bits");
        if (bits_shift < 0 || bits_shift > 20) {
            throw std::invalid_argument("bits_shift must be 0..20");
        }
        const int64_t summary_bits = (T + (int64_t{1} << bits_shift) - 1) >> bits_shift;
        if (bits.shape[2] < (summary_bits + 31) / 32) {
            throw std::invalid_argument("resident_bits needs ceil(ceil(T / 2^bits_shift) / 32) words per row");
        }
        if (counts_q_p != nullptr) {
            const ekv_tensor& groups = need(counts_q_p, "resident_counts");
            if (bits_shift == 0) {
                throw std::invalid_argument("resident_counts serve a summary with bits_shift > 0");
            }
            need_ndim(groups, 3, "resident_counts");
            need_i32(groups, "resident_counts");
            need_dim(groups, 0, L, "resident_counts");
            need_dim(groups, 1, R, "resident_counts");
            need_dim(groups, 2, summary_bits, "resident_counts");
            need_data(groups, "resident_counts");
        }
    } else if (counts_q_p != nullptr) {
        throw std::invalid_argument("resident_counts need resident_bits");
    }
    const int64_t count = selected.shape[0];
    if (L > 65535 || count > 0x7fffffff) {
        throw std::invalid_argument("too many layers or rows for one launch");
    }
    // An empty batch leaves every selection entry stray: nothing to launch
    // (the kernel's first reads assume batch row 0 exists).
    const bool launches = count > 0 && L > 0 && W > 0 && B > 0;
    if (launches) {
        for (const auto* t : {&topk, &rows, &selected, &slots, &misses, &counts, &table, &slot_token, &stamps,
                              &slot_base, &host_table, &promote_src, &promote_dst}) {
            need_data(*t, "tensor");
        }
        if (T == 0) {
            throw std::invalid_argument("the token table has no positions");   // host rows are read at position 0
        }
    }
    if (check_only()) {
        return 0;
    }
    if (!launches) {
        if (counter != nullptr) {
            advance_step_kernel<<<dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream)>>>(counter);
            check_hip(hipGetLastError(), "launch step advance");
        }
        return 0;
    }
    SwapArgs a{};
    a.topk = topk.data;
    a.topk64 = topk.dtype == EKV_INT64;
    a.topk_sl = topk.stride[0];
    a.topk_sb = topk.stride[1];
    a.topk_sk = topk.stride[2];
    a.block_size = static_cast<uint32_t>(block_size);
    a.block_div = FastDiv(static_cast<uint32_t>(block_size));
    a.rows = index_ref(rows, 0);
    a.selected = index_ref(selected, 0);
    a.slot_base = index_ref(slot_base, 0);
    a.slots = static_cast<int32_t*>(slots.data);
    a.sl_l = slots.stride[0], a.sl_b = slots.stride[1], a.sl_o = slots.stride[2];
    a.misses = static_cast<const int32_t*>(misses.data);
    a.mi_l = misses.stride[0], a.mi_b = misses.stride[1], a.mi_o = misses.stride[2];
    a.counts = static_cast<const int32_t*>(counts.data);
    a.ct_l = counts.stride[0], a.ct_b = counts.stride[1];
    a.table = table.data;
    a.table16 = table.dtype == EKV_INT16;
    a.tb_l = table.stride[0], a.tb_r = table.stride[1], a.tb_t = table.stride[2], a.table_cols = T;
    if (bits_p != nullptr) {
        a.bits = static_cast<int32_t*>(bits_p->data);
        a.bt_l = bits_p->stride[0], a.bt_r = bits_p->stride[1], a.bt_w = bits_p->stride[2];
        a.bits_shift = static_cast<uint32_t>(bits_shift);
        if (counts_q_p != nullptr) {
            a.line_counts = static_cast<int32_t*>(counts_q_p->data);
            a.lc_l = counts_q_p->stride[0], a.lc_r = counts_q_p->stride[1], a.lc_q = counts_q_p->stride[2];
        }
    }
    a.selected_count = count;
    a.status = status;
    a.slot_token = static_cast<int32_t*>(slot_token.data);
    a.st_l = slot_token.stride[0], a.st_r = slot_token.stride[1], a.st_c = slot_token.stride[2];
    a.stamps = static_cast<int32_t*>(stamps.data);
    a.sp_l = stamps.stride[0], a.sp_r = stamps.stride[1], a.sp_c = stamps.stride[2];
    a.host_table = index_ref(host_table, 0);
    a.host_table.stride = 1;
    a.host_sr = host_table.stride[0];
    a.host_st = host_table.stride[1];
    a.promote_src = static_cast<int32_t*>(promote_src.data);
    a.ps_l = promote_src.stride[0], a.ps_b = promote_src.stride[1], a.ps_o = promote_src.stride[2];
    a.promote_dst = static_cast<int32_t*>(promote_dst.data);
    a.pd_l = promote_dst.stride[0], a.pd_b = promote_dst.stride[1], a.pd_o = promote_dst.stride[2];
    a.batch = B;
    a.table_rows = R;
    a.capacity = C;
    a.width = static_cast<uint32_t>(W);
    a.step = step;
    a.step_counter = counter;
    a.hash_size = 2;
    a.hash_log2 = 1;
    while (a.hash_size < 2 * W) {
        a.hash_size <<= 1;
        ++a.hash_log2;
    }
    a.touched_words = static_cast<uint32_t>((C + 31) / 32);
    // The hash region holds 16 * hash_size bits: a bitmap of the tokens when they fit.
    a.token_bitmap = T <= int64_t{16} * a.hash_size ? 1u : 0u;
    a.bitmap_words = static_cast<uint32_t>(a.token_bitmap ? (T + 31) / 32 : 0);
    // stamps, miss tokens, touched bits, the 16-bit hash buckets (then the
    // victim list, 2 bytes per victim: at most W <= hash_size / 2), the owners
    static_assert(kMaxWidth <= 0x7fff && kMaxCapacity <= 0x7fff, "miss indices and slots fit 16 bits");
    const size_t lds = static_cast<size_t>(C) * 4 + static_cast<size_t>(W) * 4 +
                       static_cast<size_t>(a.touched_words) * 4 + static_cast<size_t>(a.hash_size) * 2 +
                       static_cast<size_t>(W) * 2;
    const dim3 grid(static_cast<uint32_t>(count), static_cast<uint32_t>(L));
    const auto s = static_cast<hipStream_t>(stream);
    // Registers per thread: 16 stamps up to C = 4096 (else 32), 8 lanes up to W = 2048 (else 16).
    const bool wide_slots = C > 16 * kThreads, wide_lanes = W > 8 * kThreads;
    auto* kernel = wide_slots ? (wide_lanes ? swap_in_kernel<32, 16> : swap_in_kernel<32, 8>)
                              : (wide_lanes ? swap_in_kernel<16, 16> : swap_in_kernel<16, 8>);
    if (lds > 64 * 1024) {
        check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                  "raise the swap-in LDS limit");
    }
    kernel<<<grid, dim3(kThreads), lds, s>>>(a);
    check_hip(hipGetLastError(), "launch swap-in");
    if (counter != nullptr) {
        advance_step_kernel<<<dim3(1), dim3(64), 0, s>>>(counter);
        check_hip(hipGetLastError(), "launch step advance");
    }
    return 0;
}

}  // namespace
}  // namespace ekv

extern "C" int ekv_swap_in(const ekv_tensor* topk, int64_t block_size, const ekv_tensor* rows,
                           const ekv_tensor* selected, const ekv_tensor* slots, const ekv_tensor* misses,
                           const ekv_tensor* miss_count, const ekv_tensor* table, const ekv_tensor* resident_bits,
                           int64_t bits_shift, const ekv_tensor* resident_counts, const ekv_tensor* slot_token,
                           const ekv_tensor* stamps,
                           const ekv_tensor* slot_base, const ekv_tensor* host_table, const ekv_tensor* promote_src,
                           const ekv_tensor* promote_dst, int64_t step, const ekv_tensor* status, void* stream) {
    return ekv::guarded(-1, [&] {
        return ekv::swap_in(topk, block_size, rows, selected, slots, misses, miss_count, table, resident_bits,
                            bits_shift, resident_counts, slot_token, stamps, slot_base, host_table, promote_src,
                            promote_dst, step, nullptr, status, stream);
    });
}

extern "C" int ekv_swap_in_counted(const ekv_tensor* topk, int64_t block_size, const ekv_tensor* rows,
                                   const ekv_tensor* selected, const ekv_tensor* slots, const ekv_tensor* misses,
                                   const ekv_tensor* miss_count, const ekv_tensor* table,
                                   const ekv_tensor* resident_bits, int64_t bits_shift,
                                   const ekv_tensor* resident_counts, const ekv_tensor* slot_token,
                                   const ekv_tensor* stamps,
                                   const ekv_tensor* slot_base, const ekv_tensor* host_table,
                                   const ekv_tensor* promote_src, const ekv_tensor* promote_dst,
                                   const ekv_tensor* step_counter, const ekv_tensor* status, void* stream) {
    return ekv::guarded(-1, [&] {
        if (step_counter == nullptr) {
            throw std::invalid_argument("step_counter is required");
        }
        return ekv::swap_in(topk, block_size, rows, selected, slots, misses, miss_count, table, resident_bits,
                            bits_shift, resident_counts, slot_token, stamps, slot_base, host_table, promote_src,
                            promote_dst, 0, step_counter, status, stream);
    });
}
