// Resident lookup with wave64 miss compaction (gfx950).
//
// Semantics: adaptive_sparse/resident_lookup.py:6-26 (Triton _resolve) and the
// torch resolver adaptive_sparse/request_residency.py:819-825, extended with a
// leading layer dimension, an optional second indirection level and an
// ordered miss list (lanes whose slot is 0 = not resident).
//
// Launch shape: one 256-thread workgroup (4 waves) per (selected row, layer).
// A row of `width` lanes is walked in chunks of 2048 lanes; wave w owns lanes
// [512w, 512w + 512) of a chunk and processes them as 8 iterations of 64
// consecutive lanes, so a wave's lane order is the row's lane order.
// Every global load is unconditional (lanes that must not read use a clamped,
// in-bounds index and their value is masked afterwards), so the 8 loads of a
// phase are in flight together instead of waiting after each one.
// Miss compaction: each iteration's misses form a 64-bit ballot; a lane's rank
// in the miss list is (misses of lower waves in this chunk) + (misses of
// earlier iterations of its wave) + mbcnt(ballot). One LDS exchange of the 4
// wave totals per chunk; no atomics, so the list order is deterministic.
//
// Two kernels share this structure:
//   resolve_single_kernel - single level (the table value is the slot), with
//     an optional residency bitmap staged in LDS: lanes whose bit is clear are
//     misses without touching their table entry;
//   resolve_mapped_kernel - two levels (table -> logical id -> mapping -> slot),
//     the reference's form.
// The decode form (single-level int16 local-slot or int32 table behind a
// residency summary, block size 1, aligned rows) takes kernels that keep the
// lane order but give each thread two contiguous 4-lane pieces (16-byte Top-K
// loads and slot stores) and assemble each chunk's miss list in LDS:
// resolve_runs_kernel, and for rows of one chunk the persistent prefetching
// forms resolve_runs_pipe_kernel and resolve_runs_pipe2_kernel (two stages:
// the next item's table reads are in flight during the current item's
// compaction; the default for summary rows of at most 1024 words).
// Recent window: decode Top-K sets concentrate on the most recent tokens, and
// lanes that gather single table entries cost one L2 request each. Both
// kernels therefore stage the table entries of the last kWindow positions
// before the row's length in LDS with coalesced 16-byte loads (two-level
// lookups only for int32 tables); lanes inside the window read LDS, lanes
// outside it read the bitmap and the table as before. Results do not depend
// on where the window lies. 1024 entries measured best on the 60-layer decode
// shapes: larger windows cost occupancy (LDS) more than they save.
#include "../../include/ekv_kernels.h"
#include "ekv_common.h"
#include "ekv_device.h"
#include "ekv_fastdiv.h"
#include "ekv_tensor_util.h"

#include <algorithm>
#include <atomic>
#include <stdexcept>
#include <type_traits>

namespace ekv {
namespace {

// Launch shape (measured best on the 60-layer decode shapes, 128 requests x
// 2048 lanes x 65,536-token tables): 256-thread workgroups walking a row in
// chunks of 8 64-lane iterations per wave; a recent window of 1024 table
// entries staged in LDS for the strided int32 form; summary rows of up to
// 4096 words staged in LDS (else lanes read their word); 32-bit byte-offset
// addressing for unit-stride rows; non-temporal Top-K loads and slot stores
// (read or written once: 3-5 % faster, and only with both, since the table
// lines that lanes of a row share keep the cache). int16 local-slot lookups
// with block size 1 and 16-byte aligned rows give each thread two contiguous
// 4-lane pieces (resolve_local_runs) instead of 8 strided 64-lane iterations.
constexpr int kThreads = 256;
constexpr int kIters = 8;                       // 64-lane iterations per wave per chunk
constexpr int kWaveSpan = 64 * kIters;          // 512 lanes per wave per chunk
constexpr int kChunkLanes = kThreads * kIters;  // 2048 lanes per chunk
constexpr int kStagedBitWords = 4096;           // 4096 words: T <= 131072 tokens
constexpr int kWindow = 1024;
static_assert(kWindow % 128 == 0, "the window must keep 16-byte alignment of the staged bitmap");
static_assert(kThreads % 64 == 0 && kThreads <= 1024, "whole waves per workgroup");

struct LookupArgs {
    const void* topk;
    int64_t topk_sl, topk_sb, topk_sk;
    const void* table;
    int64_t table_sl, table_sr, table_sc, table_rows, table_cols;
    const void* mapping;
    int64_t map_sl, map_s, map_len;
    const int32_t* bits;                 // [L?, R, W] words, bit p of a row = table[row, p] != 0
    int64_t bits_sl, bits_sr, bits_sw;
    int64_t bits_words;                  // words covering the table row: ceil(ceil(table_cols / 2^shift) / 32)
    uint32_t bits_shift;                 // bit q of a row covers positions [q << shift, (q + 1) << shift)
    IndexRef rows, lengths, selected;
    IndexRef slot_base;                  // int16 local tables: global slot of each request's local slot 0
    int32_t* out;
    int64_t out_sl, out_sb, out_so;
    int32_t* misses;
    int64_t miss_sl, miss_sb, miss_so;
    int32_t* counts;
    int64_t count_sl, count_sb;
    int64_t batch;
    int32_t window;                      // stage the recent window (int32 table)
    int32_t bits_staged;                 // stage the bitmap row in LDS
    int32_t runs;                        // int16 local form: contiguous 8-lane runs per thread
    int32_t pipe;                        // ... of one chunk, prefetching persistent form
    uint32_t width;
    uint32_t block_size;
    FastDiv block_div;
};

// Residency summaries: bit q of a row covers table positions
// [q << shift, (q + 1) << shift). shift 0 is the per-position bitmap; a
// larger shift gives one bit per group of positions (shift 6: one bit per
// 128-byte line of an int16 table). A set bit whose group holds no resident
// entry only costs that lane a table read, so a summary may be a superset.
constexpr int64_t kMaxBitsShift = 20;

// Words of a summary row over `cols` positions.
inline int64_t summary_words(int64_t cols, int64_t shift) {
    const int64_t bits = (cols + (int64_t{1} << shift) - 1) >> shift;
    return (bits + 31) / 32;
}

// Loads and stores of data touched once per launch (Top-K indices, slots),
// with the non-temporal hint.
template <typename T>
__device__ __forceinline__ T stream_load(const T* p) {
    return __builtin_nontemporal_load(p);
}

template <typename T>
__device__ __forceinline__ void stream_store(T value, T* p) {
    __builtin_nontemporal_store(value, p);
}

// Element `index` of a row at `base` with element stride `stride`. The dense
// form (stride 1 and row extents below 4 GiB, both checked on the host)
// addresses with a 32-bit byte offset from the workgroup-uniform base, so a
// lane's address takes one VGPR instead of two.
template <bool kDense, typename T>
__device__ __forceinline__ T* element(T* base, int64_t stride, uint32_t index) {
    if constexpr (kDense) {
        using Byte = std::conditional_t<std::is_const_v<T>, const char, char>;
        return reinterpret_cast<T*>(reinterpret_cast<Byte*>(base) + index * static_cast<uint32_t>(sizeof(T)));
    } else {
        return base + static_cast<int64_t>(index) * stride;
    }
}

// A table entry as a slot. int16 tables hold local slots: 0 (or a negative
// value) is not resident, v >= 1 is local slot v - 1 of the request, whose
// global slot is base + v - 1. Other tables hold the global slot itself.
template <typename TableT>
__device__ __forceinline__ int32_t entry_slot(int32_t value, int64_t base) {
    if constexpr (std::is_same_v<TableT, int16_t>) {
        return value > 0 ? static_cast<int32_t>(base + value - 1) : 0;
    } else {
        return value;
    }
}

// Staging of table windows and bitmap rows into LDS, by the whole workgroup;
// the caller synchronizes. Loads are issued in groups of 4 per thread with
// clamped (in-bounds) indices before the group's LDS stores. (Issuing every
// load of both regions before any store needs more VGPRs and measured slower
// on the 60-layer decode shapes: occupancy matters more than the saved round
// trip.)

template <typename T>
__device__ __forceinline__ bool dense_int32(const T* src, int64_t stride) {
    return sizeof(T) == 4 && stride == 1 && (reinterpret_cast<uintptr_t>(src) & 15) == 0;
}

// Any element type and stride: dst[0, n) = int32(src[j * stride]), in groups
// of 4 loads per thread.
template <typename T>
__device__ __forceinline__ void stage_words(uint32_t* dst, const T* src, int64_t stride, int64_t n) {
    for (int64_t first = 0; first < n; first += 4 * kThreads) {
        T v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t j = first + threadIdx.x + k * kThreads;
            v[k] = src[(j < n ? j : n - 1) * stride];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t j = first + threadIdx.x + k * kThreads;
            dst[j < n ? j : n - 1] = static_cast<uint32_t>(static_cast<int32_t>(v[k]));
        }
    }
}

// A dense, 16-byte aligned int32 region, 16-byte pieces in groups of 4 per
// thread. The stores go to the same in-range index as the loads (a piece
// past the end is folded back to j - n4, or to the last piece, and written
// twice with the same value): a store under `j < n4` let the compiler move
// each load into its store's branch and wait after each one. Folding to
// j - n4 rather than always to the last piece keeps the duplicate LDS stores
// of a wave on distinct addresses.
__device__ __forceinline__ void stage_vector(uint32_t* dst, const int32_t* src, int64_t n) {
    if (n <= 0) {
        return;
    }
    const int64_t n4 = n >> 2;
    // Piece j, or for j past the end a piece that is in range.
    const auto fold = [n4](int64_t j) { return j < n4 ? j : (j - n4 < n4 ? j - n4 : n4 - 1); };
    for (int64_t first = 0; first < n4; first += 4 * kThreads) {
        int4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[k] = reinterpret_cast<const int4*>(src)[fold(first + threadIdx.x + k * kThreads)];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            reinterpret_cast<int4*>(dst)[fold(first + threadIdx.x + k * kThreads)] = v[k];
        }
    }
    const int64_t t = (n4 << 2) + threadIdx.x;
    if (t < n) {
        dst[t] = static_cast<uint32_t>(src[t]);
    }
}

// Stages win_n table entries from win_src and bits_n bitmap words from
// bits_src (either count may be 0).
template <typename TableT>
__device__ __forceinline__ void stage_rows(uint32_t* win_dst, const TableT* win_src, int64_t win_stride,
                                           int64_t win_n, uint32_t* bits_dst, const int32_t* bits_src,
                                           int64_t bits_stride, int64_t bits_n) {
    const bool bits_fast = bits_n == 0 || dense_int32(bits_src, bits_stride);  // uniform
    if (win_n == 0 && bits_fast) {
        stage_vector(bits_dst, bits_src, bits_n);   // bitmap only (any table type)
        return;
    }
    if constexpr (sizeof(TableT) == 4) {
        if (bits_fast && dense_int32(win_src, win_stride)) {
            stage_vector(win_dst, reinterpret_cast<const int32_t*>(win_src), win_n);
            stage_vector(bits_dst, bits_src, bits_n);
            return;
        }
    }
    if (win_n > 0) {
        stage_words(win_dst, win_src, win_stride, win_n);
    }
    if (bits_n > 0) {
        stage_words(bits_dst, bits_src, bits_stride, bits_n);
    }
}

// The recent window of a table row: positions [start, start + count), with
// start a multiple of 128 and count <= kWindow; empty when staging is off.
struct Window {
    int64_t start = 0;
    int64_t count = 0;
};

__device__ __forceinline__ Window recent_window(const LookupArgs& a, int64_t bound, bool table_ok) {
    Window w;
    if (kWindow > 0 && a.window && table_ok && bound > 0) {
        w.start = bound > kWindow ? ((bound - kWindow) & ~int64_t{127}) : 0;
        w.count = bound - w.start < kWindow ? bound - w.start : kWindow;
    }
    return w;
}

// Top-K block ids of the 8 lanes of this thread in the current chunk.
template <bool kDense, typename TopkT>
__device__ __forceinline__ void load_blocks(const LookupArgs& a, const TopkT* topk, uint32_t first,
                                            TopkT (&block)[kIters]) {
#pragma unroll
    for (int i = 0; i < kIters; ++i) {
        const uint32_t o = first + i * 64;
        const uint32_t lane_o = o < a.width ? o : a.width - 1;
        const uint32_t b = a.block_div.div(lane_o);  // exact for block_size 1 too
        block[i] = stream_load(element<kDense>(topk, a.topk_sk, b));
    }
}

// Token position of lane o and whether it is valid and inside the table
// (valid = block >= 0 && pos < length, as in the reference, plus bounds).
// Positions of valid lanes are below the table width (< 2^31); other lanes get 0.
template <typename TopkT>
__device__ __forceinline__ uint32_t lane_position(const LookupArgs& a, uint32_t o, TopkT block, int64_t bound,
                                                  bool table_ok, bool& valid) {
    const uint32_t offset = o - a.block_div.div(o) * a.block_size;
    const int64_t p = static_cast<int64_t>(block) * a.block_size + offset;
    valid = o < a.width && block >= 0 && p < bound && table_ok;
    return valid ? static_cast<uint32_t>(p) : 0u;
}

// Output stores, then the ordered miss list of this chunk; returns the new
// running miss count of the row. Every thread of the workgroup must call it.
// A lane is a miss when its slot is 0 (invalid lanes hold -1). The ballots are
// taken twice, before and after the wave-total exchange, so no 64-bit masks
// stay live across the barrier.
template <bool kCompact, bool kDense = false>
__device__ __forceinline__ int32_t emit(const LookupArgs& a, int32_t* out, int32_t* misses, uint32_t first,
                                        const int32_t (&slot)[kIters], int32_t running, int32_t* wave_totals,
                                        int lane, int wave) {
#pragma unroll
    for (int i = 0; i < kIters; ++i) {
        const uint32_t o = first + i * 64;
        if (o < a.width) {
            stream_store(slot[i], element<kDense>(out, a.out_so, o));
        }
    }
    if constexpr (!kCompact) {
        return running;
    } else {
        int32_t wave_total = 0;
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            wave_total += __popcll(__ballot(first + i * 64 < a.width && slot[i] == 0));
        }
        if (lane == 0) {
            wave_totals[wave] = wave_total;
        }
        __syncthreads();
        int32_t rank = running;
        int32_t chunk_total = 0;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) {
            rank += w < wave ? wave_totals[w] : 0;
            chunk_total += wave_totals[w];
        }
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            const uint32_t o = first + i * 64;
            const bool miss = o < a.width && slot[i] == 0;
            const uint64_t mask = __ballot(miss);
            if (miss) {
                // Cached: a row's miss list starts and ends mid-line, and
                // non-temporal stores write such partial lines as whole bursts.
                *element<kDense>(misses, a.miss_so, static_cast<uint32_t>(rank) + lanes_below(mask)) =
                    static_cast<int32_t>(o);
            }
            rank += __popcll(mask);
        }
        __syncthreads();  // wave_totals is rewritten by the next chunk
        return running + chunk_total;
    }
}

template <typename TopkT, typename TableT, bool kBits, bool kCompact, bool kDense>
__device__ __forceinline__ void resolve_single(const LookupArgs& a) {
    // Dynamic LDS: [kWindow] staged window entries (when a.window), then the
    // staged bitmap row (when a.bits_staged), indexed by absolute word.
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ int32_t wave_totals[kThreads / 64];
    const int64_t row = a.selected.fetch(blockIdx.x);
    if (row < 0 || row >= a.batch) {
        return;  // uniform over the workgroup
    }
    const int64_t layer = blockIdx.y;
    const int64_t req = a.rows.fetch(row);
    const int64_t length = a.lengths.fetch(row);
    const bool table_ok = req >= 0 && req < a.table_rows && a.table_cols > 0;  // uniform
    const int64_t req_at = table_ok ? req : 0;
    const int64_t base = std::is_same_v<TableT, int16_t> && table_ok ? a.slot_base.fetch(req) : 0;
    const int64_t bound = length < a.table_cols ? length : a.table_cols;
    const TopkT* topk = static_cast<const TopkT*>(a.topk) + layer * a.topk_sl + row * a.topk_sb;
    const TableT* table = static_cast<const TableT*>(a.table) + layer * a.table_sl + req_at * a.table_sr;
    const int32_t* bits_row = kBits ? a.bits + layer * a.bits_sl + req_at * a.bits_sr : nullptr;
    const bool bits_in_lds = kBits && table_ok && a.bits_staged;  // uniform
    const Window win = recent_window(a, bound, table_ok);
    const int32_t* window = reinterpret_cast<const int32_t*>(lds);
    uint32_t* staged_bits = lds + (a.window ? kWindow : 0);
    int32_t* out = a.out + layer * a.out_sl + row * a.out_sb;
    int32_t* misses = kCompact ? a.misses + layer * a.miss_sl + row * a.miss_sb : nullptr;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int32_t running = 0;

    for (uint32_t chunk = 0; chunk < a.width; chunk += kChunkLanes) {
        const uint32_t first = chunk + wave * kWaveSpan + lane;
        TopkT block[kIters];
        load_blocks<kDense>(a, topk, first, block);
        if (chunk == 0 && (win.count > 0 || bits_in_lds)) {
            // Issued after the Top-K loads so all of them are in flight together.
            stage_rows(lds, table + win.start * a.table_sc, a.table_sc, win.count, staged_bits, bits_row, a.bits_sw,
                       bits_in_lds ? a.bits_words : 0);
            __syncthreads();
        }
        // Lanes inside the window take their slot from LDS; the others read
        // the bitmap (when given) and, if resident, their table entry.
        int32_t slot[kIters];
        uint32_t at[kIters];   // table position read from global memory (0 when none is needed)
        uint32_t global = 0;   // bit i: slot[i] is the global read
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            bool valid;
            const uint32_t p = lane_position(a, first + i * 64, block[i], bound, table_ok, valid);
            const int64_t rel = static_cast<int64_t>(p) - win.start;
            const bool inside = valid && rel >= 0 && rel < win.count;
            bool need = valid && !inside;
            if constexpr (kBits) {
                const uint32_t q = p >> a.bits_shift;
                const uint32_t w = inside ? 0u : q >> 5;
                const uint32_t word =
                    bits_in_lds ? staged_bits[w]
                                : (table_ok ? static_cast<uint32_t>(*element<kDense>(bits_row, a.bits_sw, w)) : 0u);
                need = need && ((word >> (q & 31)) & 1u);
            }
            slot[i] = inside ? entry_slot<TableT>(window[rel], base) : (valid ? 0 : -1);
            at[i] = need ? p : 0u;
            global |= static_cast<uint32_t>(need) << i;
        }
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            // Lanes that need no global read re-read entry 0 of the row (one
            // cached line shared by all of them) so the loads stay unconditional.
            const int32_t value =
                table_ok ? entry_slot<TableT>(static_cast<int32_t>(*element<kDense>(table, a.table_sc, at[i])), base) : 0;
            slot[i] = (global >> i) & 1u ? value : slot[i];
        }
        running = emit<kCompact, kDense>(a, out, misses, first, slot, running, wave_totals, lane, wave);
    }
    if constexpr (kCompact) {
        if (threadIdx.x == 0) {
            a.counts[layer * a.count_sl + row * a.count_sb] = running;
        }
    }
}

template <typename TopkT, typename TableT, bool kBits, bool kCompact, bool kDense>
__global__ __launch_bounds__(kThreads) void resolve_single_kernel(const LookupArgs a) {
    resolve_single<TopkT, TableT, kBits, kCompact, kDense>(a);
}

// The int16 local-slot form with its bitmap and dense rows fits 64 VGPRs, and
// only its SGPRs would hold it to 7 waves per SIMD: 8 waves measured 5 %
// faster on the 60-layer decode shapes (other forms spill at 8 waves).
template <bool kCompact>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void resolve_local_kernel(const LookupArgs a) {
    resolve_single<int32_t, int16_t, true, kCompact, true>(a);
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// The decode default (int32 Top-K, int16 local-slot table, residency bitmap,
// block size 1, dense rows) with contiguous pieces of 4 lanes per thread:
// thread t owns lanes [chunk + 4t, +4) and [chunk + 1024 + 4t, +4) of a
// 2048-lane chunk. It reads its Top-K ids and writes its slots as one 16-byte
// piece per half (the host checks that every Top-K and output row is 16-byte
// aligned and the width a multiple of 8), so each load and store instruction
// of a wave covers 1 KiB without gaps, with a quarter of the instructions of
// the strided form.
// Miss ranks: all misses of the first half precede those of the second. Per
// half, a thread's miss count (0..4) is ranked inside its wave by three
// bit-plane ballots and across waves by one LDS exchange of wave totals; a
// thread puts its misses in lane order from its rank on, so the list is the
// same ascending list as the strided form's. The chunk's list is assembled
// in LDS and then written out by consecutive threads, so its stores are
// coalesced instead of one scattered 4-byte store per miss: 11-13 % faster
// on the 60-layer decode shapes.
template <bool kCompact>
__device__ __forceinline__ void resolve_local_runs(const LookupArgs& a) {
    static_assert(kIters == 8, "two 4-lane pieces per thread");
    constexpr uint32_t kPiece = 4;
    constexpr uint32_t kHalf = kThreads * kPiece;  // 1024 lanes
    constexpr int kWaves = kThreads / 64;
    extern __shared__ __align__(16) uint32_t lds[];   // the staged bitmap row
    __shared__ int32_t wave_totals[2 * kWaves];       // [half][wave]
    __shared__ int32_t chunk_misses[kChunkLanes];
    const int64_t row = a.selected.fetch(blockIdx.x);
    if (row < 0 || row >= a.batch) {
        return;  // uniform over the workgroup
    }
    const int64_t layer = blockIdx.y;
    const int32_t* topk = static_cast<const int32_t*>(a.topk) + layer * a.topk_sl + row * a.topk_sb;
    // Top-K ids of lanes [chunk + 4t, +4) and [chunk + 1024 + 4t, +4); a thread
    // past the width re-reads the row's last piece.
    const auto load_ids = [&](uint32_t chunk, i32x4 (&ids)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t first = chunk + h * kHalf + threadIdx.x * kPiece;
            ids[h] = stream_load(reinterpret_cast<const i32x4*>(
                element<true>(topk, 1, first < a.width ? first : a.width - kPiece)));
        }
    };
    // The first chunk's ids depend on the row alone, so they are requested
    // before the request's length, table row and slot base are read.
    i32x4 ids[2];
    load_ids(0, ids);
    const int64_t req = a.rows.fetch(row);
    const int64_t length = a.lengths.fetch(row);
    const bool table_ok = req >= 0 && req < a.table_rows && a.table_cols > 0;  // uniform
    const int64_t req_at = table_ok ? req : 0;
    const int64_t base = table_ok ? a.slot_base.fetch(req) : 0;
    const int64_t bound = length < a.table_cols ? length : a.table_cols;
    const int16_t* table = static_cast<const int16_t*>(a.table) + layer * a.table_sl + req_at * a.table_sr;
    const int32_t* bits_row = a.bits + layer * a.bits_sl + req_at * a.bits_sr;
    const bool bits_in_lds = table_ok && a.bits_staged;  // uniform
    int32_t* out = a.out + layer * a.out_sl + row * a.out_sb;
    int32_t* misses = kCompact ? a.misses + layer * a.miss_sl + row * a.miss_sb : nullptr;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int32_t running = 0;

    for (uint32_t chunk = 0; chunk < a.width; chunk += kChunkLanes) {
        const uint32_t first[2] = {chunk + threadIdx.x * kPiece, chunk + kHalf + threadIdx.x * kPiece};
        const bool live[2] = {first[0] < a.width, first[1] < a.width};  // pieces are whole: width % 8 == 0
        if (chunk != 0) {
            load_ids(chunk, ids);
        }
        if (chunk == 0 && bits_in_lds) {
            // Issued after the Top-K loads so all of them are in flight together.
            stage_rows<int16_t>(nullptr, nullptr, 0, 0, lds, bits_row, a.bits_sw, a.bits_words);
            __syncthreads();
        }
        const int32_t block[kIters] = {ids[0].x, ids[0].y, ids[0].z, ids[0].w, ids[1].x, ids[1].y, ids[1].z, ids[1].w};
        int32_t slot[kIters];
        uint32_t at[kIters];   // table position to read (0 when none is needed)
        uint32_t need = 0;     // bit j: lane j reads its table entry
#pragma unroll
        for (int j = 0; j < kIters; ++j) {
            const bool valid = live[j / kPiece] && table_ok && block[j] >= 0 && block[j] < bound;
            const uint32_t p = valid ? static_cast<uint32_t>(block[j]) : 0u;
            const uint32_t q = p >> a.bits_shift;
            const uint32_t word =
                bits_in_lds ? lds[q >> 5]
                            : (table_ok ? static_cast<uint32_t>(*element<true>(bits_row, 1, q >> 5)) : 0u);
            const bool resident = valid && ((word >> (q & 31)) & 1u);
            slot[j] = valid ? 0 : -1;
            at[j] = resident ? p : 0u;
            need |= static_cast<uint32_t>(resident) << j;
        }
#pragma unroll
        for (int j = 0; j < kIters; ++j) {
            // Lanes that need no entry re-read entry 0 of the row, so the loads stay unconditional.
            const int32_t value = table_ok ? entry_slot<int16_t>(*element<true>(table, 1, at[j]), base) : 0;
            slot[j] = (need >> j) & 1u ? value : slot[j];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (live[h]) {
                stream_store(i32x4{slot[4 * h], slot[4 * h + 1], slot[4 * h + 2], slot[4 * h + 3]},
                             reinterpret_cast<i32x4*>(element<true>(out, 1, first[h])));
            }
        }
        if constexpr (kCompact) {
            uint32_t miss = 0;  // bit j: lane j is a miss
#pragma unroll
            for (int j = 0; j < kIters; ++j) {
                miss |= static_cast<uint32_t>(live[j / kPiece] && slot[j] == 0) << j;
            }
            uint32_t below[2] = {0, 0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t count = __popc((miss >> (kPiece * h)) & 0xfu);
                uint32_t wave_total = 0;
#pragma unroll
                for (int b = 0; b < 3; ++b) {
                    const uint64_t plane = __ballot((count >> b) & 1u);
                    below[h] += lanes_below(plane) << b;
                    wave_total += static_cast<uint32_t>(__popcll(plane)) << b;
                }
                if (lane == 0) {
                    wave_totals[h * kWaves + wave] = static_cast<int32_t>(wave_total);
                }
            }
            __syncthreads();
            int32_t rank[2] = {static_cast<int32_t>(below[0]), static_cast<int32_t>(below[1])};
            int32_t half_total[2] = {0, 0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    rank[h] += w < wave ? wave_totals[h * kWaves + w] : 0;
                    half_total[h] += wave_totals[h * kWaves + w];
                }
            }
            rank[1] += half_total[0];
            const int32_t chunk_total = half_total[0] + half_total[1];
#pragma unroll
            for (int j = 0; j < kIters; ++j) {
                if ((miss >> j) & 1u) {
                    const int32_t lane_id = static_cast<int32_t>(first[j / kPiece] + j % kPiece);
                    chunk_misses[rank[j / kPiece]] = lane_id;
                    ++rank[j / kPiece];
                }
            }
            __syncthreads();
            for (int32_t i = threadIdx.x; i < chunk_total; i += kThreads) {
                *element<true>(misses, 1, static_cast<uint32_t>(running + i)) = chunk_misses[i];
            }
            __syncthreads();  // wave_totals (and the staged list) are rewritten by the next chunk
            running += chunk_total;
        }
    }
    if constexpr (kCompact) {
        if (threadIdx.x == 0) {
            a.counts[layer * a.count_sl + row * a.count_sb] = running;
        }
    }
}

template <bool kCompact>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void resolve_runs_kernel(const LookupArgs a) {
    resolve_local_runs<kCompact>(a);
}

// Prefetching form of the contiguous-pieces kernel, for rows of one chunk
// (width <= 2048) whose bitmap rows are dense, 16-byte aligned and at most
// 2048 words (T <= 65536), a multiple of 4 words long. A persistent grid walks
// the (selected row, layer) items item = blockIdx.x + k * gridDim.x, at most
// kPipeMaxItems per workgroup:
//  - the index metadata of all of a workgroup's items (selected row, request
//    row, length, slot base) is read once at the start, by one thread per
//    item, into LDS, so no item waits on a chain of dependent index loads;
//  - the next item's Top-K ids and bitmap row are loaded into registers right
//    behind the current item's table reads, so they are in flight while the
//    current item's table reads, stores and miss compaction complete.
// Every load is unconditional with clamped, in-bounds addresses (a clamped
// bitmap piece is written to LDS twice with the same value), so the compiler
// cannot sink a load into the branch that consumes it and serialize the
// staging; the last iteration's loads for a next item that does not exist read
// one line of each row. Results equal the contiguous-pieces kernel's.
constexpr uint32_t kPipeBitPieces = 2 * kThreads;   // 16-byte bitmap pieces per item at most: 2048 words
constexpr uint32_t kPipeMaxItems = 16;              // items per workgroup
constexpr uint32_t kNoRow = 0xffffffffu;

// Index metadata of one item: row = kNoRow when the selected row names no
// batch row, req = kNoRow when the request has no table row.
struct RunsMeta {
    uint32_t row, req, base;   // base: low 32 bits of the request's slot base
    int32_t bound;             // positions below it are valid: min(length, T), at least 0
};

// The per-thread loads of one item: Top-K ids of lanes [4t, +4) and
// [1024 + 4t, +4), bitmap pieces t and (kBitLoads = 2) 256 + t, clamped to
// the row. Rows of at most 256 pieces (1024 words: a per-position bitmap of
// T <= 32768, or a coarser summary) take one piece per thread.
template <int kBitLoads>
struct RunsLoads {
    i32x4 ids[2];
    i32x4 bits[kBitLoads];
};

// The loads of one item. A stray selection reads batch row 0 and a request
// without a table row bitmap row 0 (in bounds, discarded). With `first_only`
// (uniform) every thread reads the first 16-byte piece of both rows: the
// workgroup's last iteration issues loads nobody uses, and one line each keeps
// them unconditional without fetching two more rows.
template <int kBitLoads>
__device__ __forceinline__ RunsLoads<kBitLoads> runs_issue(const LookupArgs& a, uint32_t layer, const RunsMeta& m,
                                                           bool first_only) {
    constexpr uint32_t kHalf = kThreads * 4;
    RunsLoads<kBitLoads> l;
    const uint32_t row = m.row != kNoRow ? m.row : 0u;
    const int32_t* topk = static_cast<const int32_t*>(a.topk) + layer * a.topk_sl + row * a.topk_sb;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t first = h * kHalf + threadIdx.x * 4;
        const uint32_t at = first_only ? 0u : (first < a.width ? first : a.width - 4);
        l.ids[h] = stream_load(reinterpret_cast<const i32x4*>(element<true>(topk, 1, at)));
    }
    const bool table_ok = m.row != kNoRow && m.req != kNoRow;
    const int32_t* row_bits = a.bits + layer * a.bits_sl + (table_ok ? m.req : 0u) * a.bits_sr;
    const uint32_t last = table_ok && !first_only ? static_cast<uint32_t>((a.bits_words + 3) >> 2) - 1 : 0u;
#pragma unroll
    for (int h = 0; h < kBitLoads; ++h) {
        const uint32_t piece = h * kThreads + threadIdx.x;
        l.bits[h] = *reinterpret_cast<const i32x4*>(element<true>(row_bits, 1, 4 * (piece < last ? piece : last)));
    }
    return l;
}

__device__ __forceinline__ RunsMeta runs_meta(const uint4* meta, uint32_t k) {
    const uint4 v = meta[k];
    return RunsMeta{v.x, v.y, v.z, static_cast<int32_t>(v.w)};
}

// TableT: int16_t (local slot + 1 per entry, plus the request's slot base) or
// int32_t (the global slot itself).
template <bool kCompact, typename TableT, int kBitLoads>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void resolve_runs_pipe_kernel(const LookupArgs a, uint32_t items, uint32_t count, FastDiv count_div) {
    constexpr uint32_t kPiece = 4;
    constexpr uint32_t kHalf = kThreads * kPiece;  // 1024 lanes
    constexpr int kWaves = kThreads / 64;
    __shared__ __align__(16) uint32_t staged_bits[4 * kThreads * kBitLoads];
    __shared__ uint4 meta[kPipeMaxItems];
    __shared__ int32_t wave_totals[2 * kWaves];   // [half][wave]
    __shared__ int32_t chunk_misses[kChunkLanes];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t first[2] = {threadIdx.x * kPiece, kHalf + threadIdx.x * kPiece};
    const bool live_piece[2] = {first[0] < a.width, first[1] < a.width};  // pieces are whole: width % 8 == 0
    const uint32_t last_piece = static_cast<uint32_t>((a.bits_words + 3) >> 2) - 1;
    const uint32_t n = (items - blockIdx.x + gridDim.x - 1) / gridDim.x;  // this workgroup's items, <= kPipeMaxItems

    if (threadIdx.x < n) {
        const uint32_t item = blockIdx.x + threadIdx.x * gridDim.x;
        const uint32_t item_layer = count_div.div(item);
        const int64_t row = a.selected.fetch(item - item_layer * count);
        const bool live = row >= 0 && row < a.batch;
        uint4 m{kNoRow, kNoRow, 0u, 0u};
        if (live) {
            const int64_t req = a.rows.fetch(row);
            const int64_t length = a.lengths.fetch(row);
            const bool table_ok = req >= 0 && req < a.table_rows && a.table_cols > 0;
            const int64_t bound = length < a.table_cols ? length : a.table_cols;
            m.x = static_cast<uint32_t>(row);
            m.y = table_ok ? static_cast<uint32_t>(req) : kNoRow;
            if constexpr (std::is_same_v<TableT, int16_t>) {
                m.z = table_ok ? static_cast<uint32_t>(a.slot_base.fetch(req)) : 0u;
            }
            m.w = static_cast<uint32_t>(bound > 0 ? static_cast<int32_t>(bound) : 0);
        }
        meta[threadIdx.x] = m;
    }
    __syncthreads();

    RunsMeta cur = runs_meta(meta, 0);
    uint32_t layer = count_div.div(blockIdx.x);
    RunsLoads<kBitLoads> loads = runs_issue<kBitLoads>(a, layer, cur, false);
    for (uint32_t k = 0;;) {
        const bool last_item = k + 1 >= n;
        const uint32_t k_next = last_item ? k : k + 1;
        const uint32_t layer_next = count_div.div(blockIdx.x + k_next * gridDim.x);
        const RunsMeta nxt = runs_meta(meta, k_next);
        RunsLoads<kBitLoads> next_loads;
        if (cur.row != kNoRow) {  // uniform
            const bool table_ok = cur.req != kNoRow;
            // Staged unconditionally (an item without a table row read summary
            // row 0, and none of its lanes is valid), so the loads are not
            // moved into a branch that waits for every load in flight.
#pragma unroll
            for (int h = 0; h < kBitLoads; ++h) {
                const uint32_t piece = h * kThreads + threadIdx.x;
                *reinterpret_cast<i32x4*>(&staged_bits[4 * (piece < last_piece ? piece : last_piece)]) = loads.bits[h];
            }
            __syncthreads();
            const int32_t block[kIters] = {loads.ids[0].x, loads.ids[0].y, loads.ids[0].z, loads.ids[0].w,
                                           loads.ids[1].x, loads.ids[1].y, loads.ids[1].z, loads.ids[1].w};
            int32_t slot[kIters];
            uint32_t at[kIters];   // table position to read (0 when none is needed)
            uint32_t need = 0;     // bit j: lane j reads its table entry
            // Bitwise, not short-circuit: every lane reads its LDS word, so
            // the reads are not split into one branch and wait per lane.
#pragma unroll
            for (int j = 0; j < kIters; ++j) {
                const bool valid = live_piece[j / kPiece] & table_ok & (block[j] >= 0) & (block[j] < cur.bound);
                const uint32_t p = valid ? static_cast<uint32_t>(block[j]) : 0u;
                const uint32_t q = p >> a.bits_shift;
                const uint32_t word = staged_bits[q >> 5];
                const bool resident = (static_cast<uint32_t>(valid) & (word >> (q & 31))) != 0u;
                slot[j] = valid ? 0 : -1;
                at[j] = resident ? p : 0u;
                need |= static_cast<uint32_t>(resident) << j;
            }
            // Lanes that need no entry re-read entry 0 of the row; without a
            // table row every lane re-reads entry 0 of row 0 of this layer.
            const TableT* table = static_cast<const TableT*>(a.table) + layer * a.table_sl +
                                  (table_ok ? cur.req : 0u) * a.table_sr;
            TableT entry[kIters];
#pragma unroll
            for (int j = 0; j < kIters; ++j) {
                entry[j] = *element<true>(table, 1, at[j]);
            }
            // The next item's loads go out behind this item's table reads.
            next_loads = runs_issue<kBitLoads>(a, layer_next, nxt, last_item);
#pragma unroll
            for (int j = 0; j < kIters; ++j) {
                const int32_t e = entry[j];
                int32_t value = e;   // int32 tables hold the slot itself
                if constexpr (std::is_same_v<TableT, int16_t>) {
                    value = e > 0 ? static_cast<int32_t>(cur.base + static_cast<uint32_t>(e) - 1u) : 0;
                }
                slot[j] = (need >> j) & 1u ? value : slot[j];
            }
            int32_t* out = a.out + layer * a.out_sl + cur.row * a.out_sb;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (live_piece[h]) {
                    stream_store(i32x4{slot[4 * h], slot[4 * h + 1], slot[4 * h + 2], slot[4 * h + 3]},
                                 reinterpret_cast<i32x4*>(element<true>(out, 1, first[h])));
                }
            }
            if constexpr (kCompact) {
                int32_t* misses = a.misses + layer * a.miss_sl + cur.row * a.miss_sb;
                uint32_t miss = 0;  // bit j: lane j is a miss
#pragma unroll
                for (int j = 0; j < kIters; ++j) {
                    miss |= static_cast<uint32_t>(live_piece[j / kPiece] && slot[j] == 0) << j;
                }
                uint32_t below[2] = {0, 0};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t c = __popc((miss >> (kPiece * h)) & 0xfu);
                    uint32_t wave_total = 0;
#pragma unroll
                    for (int b = 0; b < 3; ++b) {
                        const uint64_t plane = __ballot((c >> b) & 1u);
                        below[h] += lanes_below(plane) << b;
                        wave_total += static_cast<uint32_t>(__popcll(plane)) << b;
                    }
                    if (lane == 0) {
                        wave_totals[h * kWaves + wave] = static_cast<int32_t>(wave_total);
                    }
                }
                __syncthreads();
                int32_t rank[2] = {static_cast<int32_t>(below[0]), static_cast<int32_t>(below[1])};
                int32_t half_total[2] = {0, 0};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int w = 0; w < kWaves; ++w) {
                        rank[h] += w < wave ? wave_totals[h * kWaves + w] : 0;
                        half_total[h] += wave_totals[h * kWaves + w];
                    }
                }
                rank[1] += half_total[0];
                const int32_t total = half_total[0] + half_total[1];
#pragma unroll
                for (int j = 0; j < kIters; ++j) {
                    if ((miss >> j) & 1u) {
                        chunk_misses[rank[j / kPiece]++] = static_cast<int32_t>(first[j / kPiece] + j % kPiece);
                    }
                }
                __syncthreads();
                for (int32_t i = threadIdx.x; i < total; i += kThreads) {
                    *element<true>(misses, 1, static_cast<uint32_t>(i)) = chunk_misses[i];
                }
                if (threadIdx.x == 0) {
                    a.counts[layer * a.count_sl + cur.row * a.count_sb] = total;
                }
                // The two barriers above order this item's LDS reads before
                // the next item's writes.
            } else {
                __syncthreads();  // the staged bitmap is rewritten by the next item
            }
        } else {
            next_loads = runs_issue<kBitLoads>(a, layer_next, nxt, last_item);
        }
        if (++k >= n) {
            break;
        }
        cur = nxt;
        layer = layer_next;
        loads = next_loads;
    }
}

template <typename TopkT, typename TableT, typename MapT, bool kCompact>
__global__ __launch_bounds__(kThreads) void resolve_mapped_kernel(const LookupArgs a) {
    // Dynamic LDS: [kWindow] staged logical ids of the recent window (int32
    // tables only, so a staged id is the table value itself).
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ int32_t wave_totals[kThreads / 64];
    const int64_t layer = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // The selection entry, and the request row, length and first chunk's
    // Top-K ids of the row it names on the guess that the selection is the
    // identity (entry j names batch row j), are requested together, so the
    // table reads come after one memory level instead of two; a different
    // entry re-reads them for its row. The batch is not empty (the host
    // launches nothing for an empty one). A stray entry runs no chunk and
    // writes nothing: there is no early return, which would let the
    // compiler move the guessed loads past it and wait for them there.
    const uint32_t zero = opaque_zero();
    const int64_t guess = blockIdx.x < a.batch ? blockIdx.x : 0;
    PendingIndex entry_read = issue_index(a.selected, blockIdx.x, zero);
    PendingIndex req_read = issue_index(a.rows, guess, zero);
    PendingIndex length_read = issue_index(a.lengths, guess, zero);
    const TopkT* topk_rows = static_cast<const TopkT*>(a.topk) + layer * a.topk_sl;
    TopkT block[kIters];
    load_blocks<false>(a, topk_rows + guess * a.topk_sb, wave * kWaveSpan + lane, block);
    // One wait for all six index words: passed through one asm statement,
    // they are read back (made uniform) only after every load is issued.
    // Without it the compiler read each word back right after its load and
    // waited for it there, six round trips in a row.
    asm volatile("" : "+v"(entry_read.lo), "+v"(entry_read.hi), "+v"(req_read.lo), "+v"(req_read.hi),
                 "+v"(length_read.lo), "+v"(length_read.hi));
    const int64_t entry = index_value(a.selected, entry_read);
    const bool live = entry >= 0 && entry < a.batch;  // uniform
    const int64_t row = live ? entry : guess;
    int64_t req = index_value(a.rows, req_read);
    int64_t length = index_value(a.lengths, length_read);
    const TopkT* topk = topk_rows + row * a.topk_sb;
    if (row != guess) {  // uniform: the selection is not the identity here
        req = a.rows.fetch(row);
        length = a.lengths.fetch(row);
        load_blocks<false>(a, topk, wave * kWaveSpan + lane, block);
    }
    const uint32_t width = live ? a.width : 0u;  // a stray entry runs no chunk
    const bool table_ok = req >= 0 && req < a.table_rows && a.table_cols > 0;  // uniform
    const int64_t bound = length < a.table_cols ? length : a.table_cols;
    const TableT* table =
        static_cast<const TableT*>(a.table) + layer * a.table_sl + (table_ok ? req : 0) * a.table_sr;
    const MapT* mapping = static_cast<const MapT*>(a.mapping) + layer * a.map_sl;
    const Window win = recent_window(a, bound, table_ok);
    const int32_t* window = reinterpret_cast<const int32_t*>(lds);
    int32_t* out = a.out + layer * a.out_sl + row * a.out_sb;
    int32_t* misses = kCompact ? a.misses + layer * a.miss_sl + row * a.miss_sb : nullptr;
    int32_t running = 0;

    for (uint32_t chunk = 0; chunk < width; chunk += kChunkLanes) {
        const uint32_t first = chunk + wave * kWaveSpan + lane;
        if (chunk != 0) {
            load_blocks<false>(a, topk, first, block);
        }
        if (chunk == 0 && win.count > 0) {
            stage_rows(lds, table + win.start * a.table_sc, a.table_sc, win.count, nullptr,
                       static_cast<const int32_t*>(nullptr), 0, 0);
            __syncthreads();
        }
        uint32_t pos[kIters];
        uint32_t valid_bits = 0;   // bit i: lane i of this thread is valid
        uint32_t inside_bits = 0;  // bit i: its position lies in the staged window
        int64_t logical[kIters];
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            bool valid;
            pos[i] = lane_position(a, first + i * 64, block[i], bound, table_ok, valid);
            const int64_t rel = static_cast<int64_t>(pos[i]) - win.start;
            const bool inside = valid && rel >= 0 && rel < win.count;
            valid_bits |= static_cast<uint32_t>(valid) << i;
            inside_bits |= static_cast<uint32_t>(inside) << i;
            logical[i] = table_ok ? static_cast<int64_t>(table[(inside ? 0u : pos[i]) * a.table_sc]) : 0;
        }
        uint32_t hit_bits = 0;
        int64_t mapped[kIters];
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            if ((inside_bits >> i) & 1u) {
                logical[i] = window[static_cast<int64_t>(pos[i]) - win.start];
            }
            const bool hit = ((valid_bits >> i) & 1u) && logical[i] >= 0 && logical[i] < a.map_len;
            hit_bits |= static_cast<uint32_t>(hit) << i;
            mapped[i] = a.map_len > 0 ? static_cast<int64_t>(mapping[(hit ? logical[i] : 0) * a.map_s]) : 0;
        }
        int32_t slot[kIters];
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            slot[i] = (hit_bits >> i) & 1u ? static_cast<int32_t>(mapped[i]) : -1;
        }
        running = emit<kCompact>(a, out, misses, first, slot, running, wave_totals, lane, wave);
    }
    if constexpr (kCompact) {
        if (threadIdx.x == 0 && live) {
            a.counts[layer * a.count_sl + row * a.count_sb] = running;
        }
    }
}

// Two-stage form of the prefetching kernel (summary rows of at most 1024
// words): item k + 1's summary row is staged and its table reads are issued
// before item k's misses are compacted, so those reads (and item k + 2's
// Top-K ids and summary row, issued behind them) are in flight through item
// k's compaction barriers, which the one-stage kernel runs with only the next
// item's Top-K in flight. The summary row is staged in two LDS buffers used
// alternately: item k + 1 writes the buffer item k - 1 read, and item k - 1's
// compaction barriers separate the two. The prologue reaches the first
// item's table reads in three memory levels: the index metadata and Top-K ids
// of the first two items (guessing the identity selection), their summary
// rows, then the table entries. Its index reads are vector loads from
// clamped indices with no per-lane branch; as scalar loads and branchy reads
// they had been a chain of six or more dependent round trips (one layer per
// launch: 5.9 against 6.3 us).

// Where the two-stage kernel's threads store slot pieces that no output row
// takes (past a row's width, or of an item with no batch row): written by
// every such store, read by nothing.
__device__ i32x4 discarded_pieces[kThreads];

// One item between its two stages: its table entries in flight and its lanes'
// classification.
struct RunsPending {
    int32_t entry[kIters];
    uint32_t need;      // bit j: lane j is resident, its entry decides its slot
    uint32_t invalid;   // bit j: lane j is padding or out of range (slot -1)
};

// An item's summary row into `staged` (its first stage's barrier publishes
// it). Staged unconditionally: an item without a table row read summary row
// 0 and no lane reads it (every lane is invalid); a store under the test let
// the compiler move the summary row's load into the branch and wait there for
// every load in flight.
__device__ __forceinline__ void runs_stage(const RunsLoads<1>& loads, uint32_t* staged, uint32_t last_piece) {
    *reinterpret_cast<i32x4*>(&staged[4 * (threadIdx.x < last_piece ? threadIdx.x : last_piece)]) = loads.bits[0];
}

// First stage of an item whose summary row runs_stage has written: after a
// barrier every thread passes, classify its lanes and issue its table reads.
template <typename TableT>
__device__ __forceinline__ void runs_begin(const LookupArgs& a, uint32_t layer, const RunsMeta& m,
                                           const RunsLoads<1>& loads, uint32_t* staged,
                                           const bool (&live_piece)[2], RunsPending& p) {
    const bool table_ok = m.row != kNoRow && m.req != kNoRow;   // uniform
    __syncthreads();
    const int32_t block[kIters] = {loads.ids[0].x, loads.ids[0].y, loads.ids[0].z, loads.ids[0].w,
                                   loads.ids[1].x, loads.ids[1].y, loads.ids[1].z, loads.ids[1].w};
    uint32_t at[kIters];
    p.need = 0;
    p.invalid = 0;
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
        const bool valid = live_piece[j / 4] & table_ok & (block[j] >= 0) & (block[j] < m.bound);
        const uint32_t pos = valid ? static_cast<uint32_t>(block[j]) : 0u;
        const uint32_t q = pos >> a.bits_shift;
        const uint32_t word = staged[q >> 5];
        const bool resident = (static_cast<uint32_t>(valid) & (word >> (q & 31))) != 0u;
        at[j] = resident ? pos : 0u;
        p.need |= static_cast<uint32_t>(resident) << j;
        p.invalid |= static_cast<uint32_t>(!valid) << j;
    }
    const TableT* table =
        static_cast<const TableT*>(a.table) + layer * a.table_sl + (table_ok ? m.req : 0u) * a.table_sr;
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
        p.entry[j] = *element<true>(table, 1, at[j]);
    }
}

// The prologue's metadata of one item, level by level: its batch row (from
// the selection), then its request row and bound, then its slot base.
__device__ __forceinline__ RunsMeta meta_row(const LookupArgs& a, uint32_t item, uint32_t count,
                                             const FastDiv& count_div) {
    const uint32_t item_layer = count_div.div(item);
    const int64_t row = a.selected.fetch(item - item_layer * count);
    RunsMeta m{kNoRow, kNoRow, 0u, 0};
    if (row >= 0 && row < a.batch) {
        m.row = static_cast<uint32_t>(row);
    }
    return m;
}

__device__ __forceinline__ void meta_request(const LookupArgs& a, RunsMeta& m) {
    if (m.row != kNoRow) {
        const int64_t req = a.rows.fetch(m.row);
        const int64_t length = a.lengths.fetch(m.row);
        const bool table_ok = req >= 0 && req < a.table_rows && a.table_cols > 0;
        const int64_t bound = length < a.table_cols ? length : a.table_cols;
        m.req = table_ok ? static_cast<uint32_t>(req) : kNoRow;
        m.bound = bound > 0 ? static_cast<int32_t>(bound) : 0;
    }
}

template <typename TableT>
__device__ __forceinline__ void meta_base(const LookupArgs& a, RunsMeta& m) {
    if constexpr (std::is_same_v<TableT, int16_t>) {
        if (m.row != kNoRow && m.req != kNoRow) {
            m.base = static_cast<uint32_t>(a.slot_base.fetch(m.req));
        }
    }
}

// The request row and bound of item metadata whose batch row is known.
__device__ __forceinline__ void meta_apply(const LookupArgs& a, RunsMeta& m, int64_t req, int64_t length) {
    if (m.row != kNoRow) {
        const bool table_ok = req >= 0 && req < a.table_rows && a.table_cols > 0;
        const int64_t bound = length < a.table_cols ? length : a.table_cols;
        m.req = table_ok ? static_cast<uint32_t>(req) : kNoRow;
        m.bound = bound > 0 ? static_cast<int32_t>(bound) : 0;
    }
}

// runs_issue in two parts: the Top-K ids need only the batch row, the
// summary row needs the request.
__device__ __forceinline__ void runs_issue_ids(const LookupArgs& a, uint32_t layer, const RunsMeta& m,
                                               bool first_only, RunsLoads<1>& l) {
    constexpr uint32_t kHalf = kThreads * 4;
    const uint32_t row = m.row != kNoRow ? m.row : 0u;
    const int32_t* topk = static_cast<const int32_t*>(a.topk) + layer * a.topk_sl + row * a.topk_sb;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t first = h * kHalf + threadIdx.x * 4;
        const uint32_t at = first_only ? 0u : (first < a.width ? first : a.width - 4);
        l.ids[h] = stream_load(reinterpret_cast<const i32x4*>(element<true>(topk, 1, at)));
    }
}

// Keeps a guessed item's metadata and Top-K loads when its selection entry
// names the guessed row; otherwise re-reads them for the row the entry names
// (none for an entry outside the batch: every lane of the item is invalid).
__device__ __forceinline__ void settle_guess(const LookupArgs& a, uint32_t layer, int64_t entry, bool first_only,
                                             RunsMeta& m, RunsLoads<1>& l) {
    const uint32_t row = entry >= 0 && entry < a.batch ? static_cast<uint32_t>(entry) : kNoRow;
    if (row != m.row) {   // uniform
        m = RunsMeta{row, kNoRow, 0u, 0};
        meta_request(a, m);
        runs_issue_ids(a, layer, m, first_only, l);
    }
}

__device__ __forceinline__ void runs_issue_bits(const LookupArgs& a, uint32_t layer, const RunsMeta& m,
                                                bool first_only, RunsLoads<1>& l) {
    const bool table_ok = m.row != kNoRow && m.req != kNoRow;
    const int32_t* row_bits = a.bits + layer * a.bits_sl + (table_ok ? m.req : 0u) * a.bits_sr;
    const uint32_t last = table_ok && !first_only ? static_cast<uint32_t>((a.bits_words + 3) >> 2) - 1 : 0u;
    const uint32_t piece = threadIdx.x;
    l.bits[0] = *reinterpret_cast<const i32x4*>(element<true>(row_bits, 1, 4 * (piece < last ? piece : last)));
}

template <bool kCompact, typename TableT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void resolve_runs_pipe2_kernel(const LookupArgs a, uint32_t items, uint32_t count, FastDiv count_div) {
    constexpr uint32_t kPiece = 4;
    constexpr uint32_t kHalf = kThreads * kPiece;  // 1024 lanes
    constexpr int kWaves = kThreads / 64;
    __shared__ __align__(16) uint32_t staged_bits[2][4 * kThreads];
    __shared__ uint4 meta[kPipeMaxItems];
    __shared__ int32_t wave_totals[2 * kWaves];   // [half][wave]
    __shared__ int32_t chunk_misses[kChunkLanes];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t first[2] = {threadIdx.x * kPiece, kHalf + threadIdx.x * kPiece};
    const bool live_piece[2] = {first[0] < a.width, first[1] < a.width};  // pieces are whole: width % 8 == 0
    const uint32_t last_piece = static_cast<uint32_t>((a.bits_words + 3) >> 2) - 1;
    const uint32_t n = (items - blockIdx.x + gridDim.x - 1) / gridDim.x;  // this workgroup's items, <= kPipeMaxItems

    // Prologue. Items 0 and 1 guess the identity selection (entry j names
    // batch row j: every batch row, the decode default), so their selection
    // entries, the guessed rows' request rows and lengths and their Top-K ids
    // are requested at once; settle_guess re-reads them for the row an entry
    // actually names when it differs. Then their summary rows and slot bases.
    // Thread t reads item t's selection entry beside them, its request row and
    // length beside the summary rows, and its slot base after the first
    // item's table reads are issued (vector loads complete in issue order, so
    // waiting for it then waits for nothing the first item does not need
    // next); item t's metadata goes to LDS for the later iterations, published
    // by the next first stage's barrier. Every per-thread read is
    // unconditional, from a clamped index: a read under a per-lane condition
    // let the compiler wait for all loads in flight inside that branch.
    const uint32_t k_next = n > 1 ? 1u : 0u;
    const uint32_t k_mine = threadIdx.x < n ? threadIdx.x : 0u;
    uint32_t layer = count_div.div(blockIdx.x);
    uint32_t layer_next = count_div.div(blockIdx.x + k_next * gridDim.x);
    const uint32_t zero = opaque_zero();
    const uint32_t item_next = blockIdx.x + k_next * gridDim.x;
    const uint32_t item_mine = blockIdx.x + k_mine * gridDim.x;
    const uint32_t j_cur = blockIdx.x - layer * count, j_next = item_next - layer_next * count;
    const uint32_t j_mine = item_mine - count_div.div(item_mine) * count;
    RunsMeta cur{j_cur < a.batch ? j_cur : kNoRow, kNoRow, 0u, 0};
    RunsMeta nxt{j_next < a.batch ? j_next : kNoRow, kNoRow, 0u, 0};
    const PendingIndex entry_cur = issue_index(a.selected, j_cur, zero);
    const PendingIndex entry_next = issue_index(a.selected, j_next, zero);
    const PendingIndex req_cur = issue_index(a.rows, cur.row != kNoRow ? cur.row : 0u, zero);
    const PendingIndex len_cur = issue_index(a.lengths, cur.row != kNoRow ? cur.row : 0u, zero);
    const PendingIndex req_next = issue_index(a.rows, nxt.row != kNoRow ? nxt.row : 0u, zero);
    const PendingIndex len_next = issue_index(a.lengths, nxt.row != kNoRow ? nxt.row : 0u, zero);
    const PendingIndex entry_mine = issue_index(a.selected, j_mine, zero);
    RunsLoads<1> first_loads;
    RunsLoads<1> next_loads;
    runs_issue_ids(a, layer, cur, false, first_loads);
    runs_issue_ids(a, layer_next, nxt, n <= 1, next_loads);
    meta_apply(a, cur, index_value(a.rows, req_cur), index_value(a.lengths, len_cur));
    meta_apply(a, nxt, index_value(a.rows, req_next), index_value(a.lengths, len_next));
    settle_guess(a, layer, index_value(a.selected, entry_cur), false, cur, first_loads);
    settle_guess(a, layer_next, index_value(a.selected, entry_next), n <= 1, nxt, next_loads);
    runs_issue_bits(a, layer, cur, false, first_loads);
    runs_issue_bits(a, layer_next, nxt, n <= 1, next_loads);
    PendingIndex base_cur{0, 0}, base_next{0, 0};
    if constexpr (std::is_same_v<TableT, int16_t>) {
        base_cur = issue_index(a.slot_base, cur.req != kNoRow ? cur.req : 0u, zero);
        base_next = issue_index(a.slot_base, nxt.req != kNoRow ? nxt.req : 0u, zero);
    }
    const int64_t row_mine = lane_value(a.selected, entry_mine);
    RunsMeta mine{row_mine >= 0 && row_mine < a.batch ? static_cast<uint32_t>(row_mine) : kNoRow, kNoRow, 0u, 0};
    const PendingIndex req_mine = issue_index(a.rows, mine.row != kNoRow ? mine.row : 0u, zero);
    const PendingIndex len_mine = issue_index(a.lengths, mine.row != kNoRow ? mine.row : 0u, zero);
    RunsPending pend;
    runs_stage(first_loads, staged_bits[0], last_piece);
    runs_begin<TableT>(a, layer, cur, first_loads, staged_bits[0], live_piece, pend);
    meta_apply(a, mine, lane_value(a.rows, req_mine), lane_value(a.lengths, len_mine));
    if constexpr (std::is_same_v<TableT, int16_t>) {
        const PendingIndex base_mine = issue_index(a.slot_base, mine.req != kNoRow ? mine.req : 0u, zero);
        cur.base = cur.req != kNoRow ? static_cast<uint32_t>(index_value(a.slot_base, base_cur)) : 0u;
        nxt.base = nxt.req != kNoRow ? static_cast<uint32_t>(index_value(a.slot_base, base_next)) : 0u;
        mine.base = mine.req != kNoRow ? static_cast<uint32_t>(lane_value(a.slot_base, base_mine)) : 0u;
    }
    if (threadIdx.x < n) {   // read from the second item on, after the next first stage's barrier
        meta[threadIdx.x] = uint4{mine.row, mine.req, mine.base, static_cast<uint32_t>(mine.bound)};
    }
    for (uint32_t k = 0;; ++k) {
        // Item k's slots from its table entries.
        int32_t slot[kIters];
#pragma unroll
        for (int j = 0; j < kIters; ++j) {
            const int32_t e = pend.entry[j];
            int32_t value = e;   // int32 tables hold the slot itself
            if constexpr (std::is_same_v<TableT, int16_t>) {
                value = e > 0 ? static_cast<int32_t>(cur.base + static_cast<uint32_t>(e) - 1u) : 0;
            }
            slot[j] = (pend.need >> j) & 1u ? value : ((pend.invalid >> j) & 1u ? -1 : 0);
        }
        // The next item's summary row is staged before this item's slots are
        // stored, so waiting for it does not wait for those stores too; with
        // no next item the loads of the last iteration (one piece of row 0)
        // go to the buffer no later item reads.
        const bool more = k + 1 < n;   // uniform
        runs_stage(next_loads, staged_bits[(k + 1) & 1], last_piece);
        const bool live = cur.row != kNoRow;   // uniform
        {
            // Two stores on every path: a piece past the row or of an item
            // with no batch row goes to a scratch word block nobody reads. With
            // conditional stores the compiler could not count the stores in
            // flight and waited for all of them (their acknowledgements)
            // before staging the next item's summary row.
            int32_t* out = a.out + layer * a.out_sl + (live ? cur.row : 0u) * a.out_sb;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                i32x4* to = live && live_piece[h] ? reinterpret_cast<i32x4*>(element<true>(out, 1, first[h]))
                                                  : &discarded_pieces[threadIdx.x];
                stream_store(i32x4{slot[4 * h], slot[4 * h + 1], slot[4 * h + 2], slot[4 * h + 3]}, to);
            }
        }
        uint32_t miss = 0;  // bit j: lane j is a miss
        if constexpr (kCompact) {
#pragma unroll
            for (int j = 0; j < kIters; ++j) {
                miss |= static_cast<uint32_t>(live && live_piece[j / kPiece] && slot[j] == 0) << j;
            }
        }
        // Stage one of item k + 1 and the loads of item k + 2, ahead of item k's compaction.
        RunsMeta after = nxt;
        uint32_t layer_after = layer_next;
        RunsLoads<1> after_loads = next_loads;
        if (more) {
            runs_begin<TableT>(a, layer_next, nxt, next_loads, staged_bits[(k + 1) & 1], live_piece, pend);
            const uint32_t k_after = k + 2 < n ? k + 2 : k + 1;
            after = runs_meta(meta, k_after);
            layer_after = count_div.div(blockIdx.x + k_after * gridDim.x);
            after_loads = runs_issue<1>(a, layer_after, after, k + 2 >= n);
        }
        if constexpr (kCompact) {
            uint32_t below[2] = {0, 0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t c = __popc((miss >> (kPiece * h)) & 0xfu);
                uint32_t wave_total = 0;
#pragma unroll
                for (int b = 0; b < 3; ++b) {
                    const uint64_t plane = __ballot((c >> b) & 1u);
                    below[h] += lanes_below(plane) << b;
                    wave_total += static_cast<uint32_t>(__popcll(plane)) << b;
                }
                if (lane == 0) {
                    wave_totals[h * kWaves + wave] = static_cast<int32_t>(wave_total);
                }
            }
            __syncthreads();
            int32_t rank[2] = {static_cast<int32_t>(below[0]), static_cast<int32_t>(below[1])};
            int32_t half_total[2] = {0, 0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    rank[h] += w < wave ? wave_totals[h * kWaves + w] : 0;
                    half_total[h] += wave_totals[h * kWaves + w];
                }
            }
            rank[1] += half_total[0];
            const int32_t total = half_total[0] + half_total[1];
#pragma unroll
            for (int j = 0; j < kIters; ++j) {
                if ((miss >> j) & 1u) {
                    chunk_misses[rank[j / kPiece]++] = static_cast<int32_t>(first[j / kPiece] + j % kPiece);
                }
            }
            __syncthreads();
            if (live) {
                int32_t* misses = a.misses + layer * a.miss_sl + cur.row * a.miss_sb;
                for (int32_t i = threadIdx.x; i < total; i += kThreads) {
                    *element<true>(misses, 1, static_cast<uint32_t>(i)) = chunk_misses[i];
                }
                if (threadIdx.x == 0) {
                    a.counts[layer * a.count_sl + cur.row * a.count_sb] = total;
                }
            }
            // The two barriers above also separate item k's reads of its
            // staged summary from item k + 2's writes to the same buffer.
        } else {
            __syncthreads();   // ... which this barrier does without compaction
        }
        if (!more) {
            break;
        }
        cur = nxt;
        layer = layer_next;
        nxt = after;
        layer_next = layer_after;
        next_loads = after_loads;
    }
}

// Workgroups of the prefetching kernel resident on the whole device at once,
// per device (0 = not yet queried).
template <bool kCompact, typename TableT, int kBitLoads>
uint32_t runs_pipe_resident() {
    static std::atomic<uint32_t> resident[64];
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    if (device < 0 || device >= 64) {
        throw std::runtime_error("device ordinal out of range");
    }
    uint32_t known = resident[device].load(std::memory_order_relaxed);
    if (known == 0) {
        int per_cu = 0, cus = 0;
        check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                      &per_cu, reinterpret_cast<const void*>(resolve_runs_pipe_kernel<kCompact, TableT, kBitLoads>),
                      kThreads, 0),
                  "hipOccupancyMaxActiveBlocksPerMultiprocessor");
        check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                  "hipDeviceGetAttribute");
        known = static_cast<uint32_t>(std::max(1, per_cu) * std::max(1, cus));
        resident[device].store(known, std::memory_order_relaxed);
    }
    return known;
}

// Workgroups of the two-stage kernel resident on the whole device at once.
template <bool kCompact, typename TableT>
uint32_t runs_pipe2_resident() {
    static std::atomic<uint32_t> resident[64];
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    if (device < 0 || device >= 64) {
        throw std::runtime_error("device ordinal out of range");
    }
    uint32_t known = resident[device].load(std::memory_order_relaxed);
    if (known == 0) {
        int per_cu = 0, cus = 0;
        check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                      &per_cu, reinterpret_cast<const void*>(resolve_runs_pipe2_kernel<kCompact, TableT>), kThreads, 0),
                  "hipOccupancyMaxActiveBlocksPerMultiprocessor");
        check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                  "hipDeviceGetAttribute");
        known = static_cast<uint32_t>(std::max(1, per_cu) * std::max(1, cus));
        resident[device].store(known, std::memory_order_relaxed);
    }
    return known;
}

template <bool kCompact, typename TableT>
void launch_runs_pipe2(const LookupArgs& a, dim3 grid, hipStream_t stream) {
    const uint32_t count = grid.x;
    const uint32_t items = grid.x * grid.y;   // below 2^31 (checked by the host)
    const uint32_t groups = std::min(items, std::max(runs_pipe2_resident<kCompact, TableT>(),
                                                     (items + kPipeMaxItems - 1) / kPipeMaxItems));
    resolve_runs_pipe2_kernel<kCompact, TableT><<<dim3(groups), dim3(kThreads), 0, stream>>>(a, items, count,
                                                                                            FastDiv(count));
}

template <bool kCompact, typename TableT, int kBitLoads>
void launch_runs_pipe_loads(const LookupArgs& a, dim3 grid, hipStream_t stream) {
    const uint32_t count = grid.x;
    const uint32_t items = grid.x * grid.y;   // below 2^31 (checked by the host)
    // Resident workgroups, or more when they would take over kPipeMaxItems items each.
    const uint32_t groups = std::min(items, std::max(runs_pipe_resident<kCompact, TableT, kBitLoads>(),
                                                     (items + kPipeMaxItems - 1) / kPipeMaxItems));
    resolve_runs_pipe_kernel<kCompact, TableT, kBitLoads><<<dim3(groups), dim3(kThreads), 0, stream>>>(
        a, items, count, FastDiv(count));
}

// Summary rows of at most kThreads 16-byte pieces take the two-stage kernel;
// longer ones (up to 2 * kThreads pieces) the one-stage kernel with two
// pieces per thread.
template <bool kCompact, typename TableT>
void launch_runs_pipe(const LookupArgs& a, dim3 grid, hipStream_t stream) {
    if ((a.bits_words + 3) / 4 <= kThreads) {
        launch_runs_pipe2<kCompact, TableT>(a, grid, stream);
    } else {
        launch_runs_pipe_loads<kCompact, TableT, 2>(a, grid, stream);
    }
}

template <typename TopkT, typename TableT>
void launch_with_table(const LookupArgs& a, int32_t map_dtype, bool compact, bool dense, dim3 grid,
                       hipStream_t stream) {
    const dim3 block(kThreads);
    const size_t lds = sizeof(uint32_t) * ((a.window ? kWindow : 0) + (a.bits_staged ? a.bits_words : 0));
    if (a.mapping == nullptr) {
        const bool bits = a.bits != nullptr;
        if (dense) {
            if constexpr (std::is_same_v<TopkT, int32_t> && std::is_same_v<TableT, int16_t>) {
                if (bits && a.pipe) {
                    if (compact) {
                        launch_runs_pipe<true, int16_t>(a, grid, stream);
                    } else {
                        launch_runs_pipe<false, int16_t>(a, grid, stream);
                    }
                    return;
                }
                if (bits && a.runs) {
                    if (compact) {
                        resolve_runs_kernel<true><<<grid, block, lds, stream>>>(a);
                    } else {
                        resolve_runs_kernel<false><<<grid, block, lds, stream>>>(a);
                    }
                    return;
                }
                if (bits) {
                    if (compact) {
                        resolve_local_kernel<true><<<grid, block, lds, stream>>>(a);
                    } else {
                        resolve_local_kernel<false><<<grid, block, lds, stream>>>(a);
                    }
                    return;
                }
            }
            if constexpr (std::is_same_v<TopkT, int32_t> && std::is_same_v<TableT, int32_t>) {
                if (bits && a.pipe) {
                    if (compact) {
                        launch_runs_pipe<true, int32_t>(a, grid, stream);
                    } else {
                        launch_runs_pipe<false, int32_t>(a, grid, stream);
                    }
                    return;
                }
            }
            if (bits && compact) {
                resolve_single_kernel<TopkT, TableT, true, true, true><<<grid, block, lds, stream>>>(a);
            } else if (bits) {
                resolve_single_kernel<TopkT, TableT, true, false, true><<<grid, block, lds, stream>>>(a);
            } else if (compact) {
                resolve_single_kernel<TopkT, TableT, false, true, true><<<grid, block, lds, stream>>>(a);
            } else {
                resolve_single_kernel<TopkT, TableT, false, false, true><<<grid, block, lds, stream>>>(a);
            }
        } else if (bits && compact) {
            resolve_single_kernel<TopkT, TableT, true, true, false><<<grid, block, lds, stream>>>(a);
        } else if (bits) {
            resolve_single_kernel<TopkT, TableT, true, false, false><<<grid, block, lds, stream>>>(a);
        } else if (compact) {
            resolve_single_kernel<TopkT, TableT, false, true, false><<<grid, block, lds, stream>>>(a);
        } else {
            resolve_single_kernel<TopkT, TableT, false, false, false><<<grid, block, lds, stream>>>(a);
        }
    } else if constexpr (!std::is_same_v<TableT, int16_t>) {  // local tables are single level
        if (map_dtype == EKV_INT64) {
            if (compact) {
                resolve_mapped_kernel<TopkT, TableT, int64_t, true><<<grid, block, lds, stream>>>(a);
            } else {
                resolve_mapped_kernel<TopkT, TableT, int64_t, false><<<grid, block, lds, stream>>>(a);
            }
        } else {
            if (compact) {
                resolve_mapped_kernel<TopkT, TableT, int32_t, true><<<grid, block, lds, stream>>>(a);
            } else {
                resolve_mapped_kernel<TopkT, TableT, int32_t, false><<<grid, block, lds, stream>>>(a);
            }
        }
    }
}

template <typename TopkT>
void launch_table(const LookupArgs& a, int32_t table_dtype, int32_t map_dtype, bool compact, bool dense, dim3 grid,
                  hipStream_t stream) {
    if (table_dtype == EKV_INT64) {
        launch_with_table<TopkT, int64_t>(a, map_dtype, compact, dense, grid, stream);
    } else if (table_dtype == EKV_INT16) {
        launch_with_table<TopkT, int16_t>(a, map_dtype, compact, dense, grid, stream);
    } else {
        launch_with_table<TopkT, int32_t>(a, map_dtype, compact, dense, grid, stream);
    }
}

int resolve_resident(const ekv_tensor* topk_p, const ekv_tensor* table_p, const ekv_tensor* mapping_p,
                     const ekv_tensor* rows_p, const ekv_tensor* lengths_p, const ekv_tensor* selected_p,
                     const ekv_tensor* output_p, const ekv_tensor* misses_p, const ekv_tensor* counts_p,
                     const ekv_tensor* bits_p, int64_t block_size, void* stream,
                     const ekv_tensor* slot_base_p = nullptr, int64_t bits_shift = 0) {
    const ekv_tensor& topk = need(topk_p, "topk");
    const ekv_tensor& table = need(table_p, "table");
    const ekv_tensor& rows = need(rows_p, "rows");
    const ekv_tensor& lengths = need(lengths_p, "lengths");
    const ekv_tensor& selected = need(selected_p, "selected");
    const ekv_tensor& output = need(output_p, "output");
    need_ndim(topk, 3, "topk");
    need_index(topk, "topk");
    const int64_t layers = topk.shape[0];
    const int64_t batch = topk.shape[1];
    const int64_t k = topk.shape[2];
    if (block_size < 1) {
        throw std::invalid_argument("block_size must be positive");
    }
    const int64_t width = k * block_size;
    need_ndim(output, 3, "output");
    if (output.dtype != EKV_INT32) {
        throw std::invalid_argument("output must be int32");
    }
    need_dim(output, 0, layers, "output");
    need_dim(output, 1, batch, "output");
    need_dim(output, 2, width, "output");
    if (table.ndim != 2 && table.ndim != 3) {
        throw std::invalid_argument("table must be [R, T] or [L, R, T]");
    }
    const bool local = slot_base_p != nullptr;
    if (local) {
        if (table.dtype != EKV_INT16 || mapping_p != nullptr) {
            throw std::invalid_argument("a local-slot table is int16 and single level (mapping = NULL)");
        }
    } else {
        need_index(table, "table");
    }
    const bool layered_table = table.ndim == 3;
    if (layered_table) {
        need_dim(table, 0, layers, "table");
    }
    for (const auto* one : {&rows, &lengths, &selected}) {
        need_ndim(*one, 1, "rows/lengths/selected");
        need_index(*one, "rows/lengths/selected");
    }
    need_dim(rows, 0, batch, "rows");
    need_dim(lengths, 0, batch, "lengths");
    if (local) {
        const ekv_tensor& base = need(slot_base_p, "slot_base");
        need_ndim(base, 1, "slot_base");
        need_index(base, "slot_base");
        need_dim(base, 0, table.shape[layered_table ? 1 : 0], "slot_base");
        need_data(base, "slot_base");
    }
    const ekv_tensor* mapping = nullptr;
    if (mapping_p != nullptr) {
        mapping = &need(mapping_p, "mapping");
        need_index(*mapping, "mapping");
        if (mapping->ndim == 2) {
            need_dim(*mapping, 0, layers, "mapping");
        } else if (mapping->ndim != 1) {
            throw std::invalid_argument("mapping must be [N] or [L, N]");
        }
    }
    if (bits_p != nullptr) {
        const ekv_tensor& bits = need(bits_p, "resident_bits");
        if (mapping_p != nullptr) {
            throw std::invalid_argument("resident_bits needs the single-level form (mapping = NULL)");
        }
        if (bits.dtype != EKV_INT32 || bits.ndim != table.ndim) {
            throw std::invalid_argument("resident_bits must be int32 with the table's number of dimensions");
        }
        if (layered_table) {
            need_dim(bits, 0, layers, "resident_bits");
        }
        const int d = layered_table ? 1 : 0;
        need_dim(bits, d, table.shape[d], "resident_bits");
        if (bits_shift < 0 || bits_shift > kMaxBitsShift) {
            throw std::invalid_argument("bits_shift must be 0.." + std::to_string(kMaxBitsShift));
        }
        if (bits.shape[d + 1] < summary_words(table.shape[d + 1], bits_shift)) {
            throw std::invalid_argument("resident_bits needs ceil(ceil(T / 2^bits_shift) / 32) words per row");
        }
        need_data(bits, "resident_bits");
    }
    if ((misses_p == nullptr) != (counts_p == nullptr)) {
        throw std::invalid_argument("misses and miss_count must be given together");
    }
    const bool compact = misses_p != nullptr;
    if (compact) {
        const ekv_tensor& misses = need(misses_p, "misses");
        const ekv_tensor& counts = need(counts_p, "miss_count");
        need_ndim(misses, 3, "misses");
        need_ndim(counts, 2, "miss_count");
        if (misses.dtype != EKV_INT32 || counts.dtype != EKV_INT32) {
            throw std::invalid_argument("misses and miss_count must be int32");
        }
        need_dim(misses, 0, layers, "misses");
        need_dim(misses, 1, batch, "misses");
        need_dim(misses, 2, width, "misses");
        need_dim(counts, 0, layers, "miss_count");
        need_dim(counts, 1, batch, "miss_count");
    }
    const int64_t count = selected.shape[0];
    if (count == 0 || width == 0 || layers == 0) {
        return 0;  // the reference returns without launching
    }
    if (batch == 0) {
        return 0;  // every selection entry is stray: nothing is written (the kernels read batch row 0 first)
    }
    if (width >= (int64_t{1} << 31) - kChunkLanes) {
        throw std::invalid_argument("K * block_size must be below 2^31");
    }
    if (layers > 65535) {
        throw std::invalid_argument("at most 65535 layers per launch");
    }
    if (count > 0x7fffffff) {
        throw std::invalid_argument("too many selected rows");
    }
    for (const auto* one : {&topk, &table, &rows, &lengths, &selected, &output}) {
        need_data(*one, "tensor");
    }

    LookupArgs a{};
    a.topk = topk.data;
    a.topk_sl = topk.stride[0];
    a.topk_sb = topk.stride[1];
    a.topk_sk = topk.stride[2];
    a.table = table.data;
    const int d = layered_table ? 1 : 0;
    a.table_sl = layered_table ? table.stride[0] : 0;
    a.table_sr = table.stride[d];
    a.table_sc = table.stride[d + 1];
    a.table_rows = table.shape[d];
    a.table_cols = table.shape[d + 1];
    if (mapping != nullptr) {
        need_data(*mapping, "mapping");
        a.mapping = mapping->data;
        a.map_sl = mapping->ndim == 2 ? mapping->stride[0] : 0;
        a.map_s = mapping->stride[mapping->ndim - 1];
        a.map_len = mapping->shape[mapping->ndim - 1];
    }
    if (bits_p != nullptr) {
        const int d = layered_table ? 1 : 0;
        a.bits = static_cast<const int32_t*>(bits_p->data);
        a.bits_sl = layered_table ? bits_p->stride[0] : 0;
        a.bits_sr = bits_p->stride[d];
        a.bits_sw = bits_p->stride[d + 1];
        a.bits_words = summary_words(a.table_cols, bits_shift);
        a.bits_shift = static_cast<uint32_t>(bits_shift);
    }
    a.rows = index_ref(rows, 0);
    a.lengths = index_ref(lengths, 0);
    a.selected = index_ref(selected, 0);
    if (local) {
        a.slot_base = index_ref(*slot_base_p, 0);
    }
    a.out = static_cast<int32_t*>(output.data);
    a.out_sl = output.stride[0];
    a.out_sb = output.stride[1];
    a.out_so = output.stride[2];
    if (compact) {
        a.misses = static_cast<int32_t*>(misses_p->data);
        a.miss_sl = misses_p->stride[0];
        a.miss_sb = misses_p->stride[1];
        a.miss_so = misses_p->stride[2];
        a.counts = static_cast<int32_t*>(counts_p->data);
        a.count_sl = counts_p->stride[0];
        a.count_sb = counts_p->stride[1];
        if (a.misses == nullptr || a.counts == nullptr) {
            throw std::invalid_argument("misses / miss_count have null data pointers");
        }
    }
    a.batch = batch;
    a.width = static_cast<uint32_t>(width);
    a.block_size = static_cast<uint32_t>(block_size);
    if (block_size >= (int64_t{1} << 31)) {
        throw std::invalid_argument("block_size must be below 2^31");
    }
    if (a.table_cols >= (int64_t{1} << 31)) {
        throw std::invalid_argument("tables wider than 2^31 - 1 positions are not supported");
    }
    a.block_div = FastDiv(static_cast<uint32_t>(block_size));
    // Staging the window reads kWindow entries per (row, layer); it pays once a
    // row has at least a quarter as many lanes. Two-level lookups stage only
    // int32 tables (a staged int32 id must equal the table value).
    // int16 (local-slot) tables take no window: their per-lane 2-byte reads
    // measured faster on the 60-layer decode shapes than staging them.
    a.window = kWindow > 0 && width >= kWindow / 4 && table.dtype != EKV_INT16 &&
                       (mapping == nullptr || table.dtype == EKV_INT32) ? 1 : 0;
    a.bits_staged = bits_p != nullptr && a.bits_words <= kStagedBitWords ? 1 : 0;

    const dim3 grid(static_cast<uint32_t>(count), static_cast<uint32_t>(layers));
    const auto s = static_cast<hipStream_t>(stream);
    const int32_t map_dtype = mapping ? mapping->dtype : 0;
    // Dense rows (unit inner strides, every row extent below 4 GiB) take the
    // 32-bit byte-offset addressing of element<true>.
    constexpr int64_t kFourGiB = int64_t{1} << 32;
    const bool dense = a.topk_sk == 1 && a.table_sc == 1 && a.out_so == 1 && (!compact || a.miss_so == 1) &&
                       (a.bits == nullptr || a.bits_sw == 1) && k * itemsize(topk.dtype) < kFourGiB &&
                       a.table_cols * itemsize(table.dtype) < kFourGiB && width * 4 < kFourGiB &&
                       a.bits_words * 4 < kFourGiB;
    // Contiguous runs (dense int16 local form with a bitmap, block size 1): every
    // Top-K and output row starts 16-byte aligned and holds whole 8-lane runs.
    const auto rows_aligned = [](const void* data, int64_t s0, int64_t n0, int64_t s1, int64_t n1) {
        return (reinterpret_cast<uintptr_t>(data) & 15) == 0 && (n0 <= 1 || s0 % 4 == 0) && (n1 <= 1 || s1 % 4 == 0);
    };
    const bool pieces_layout = bits_p != nullptr && topk.dtype == EKV_INT32 && block_size == 1 &&
                               width % kIters == 0 && rows_aligned(topk.data, a.topk_sl, layers, a.topk_sb, batch) &&
                               rows_aligned(output.data, a.out_sl, layers, a.out_sb, batch);
    a.runs = local && pieces_layout ? 1 : 0;
    // The prefetching form: rows of one chunk, a non-empty batch and table
    // (stray selections and requests read batch row 0 and table entry 0 of
    // row 0, and discard them), fewer than 2^31 items, and bitmap rows of at
    // most 2048 words that start 16-byte aligned and whose tensor covers
    // ceil(words / 4) whole 16-byte pieces (the staging reads whole pieces;
    // build_residency_bits pads rows that way).
    const int64_t bits_pieces_needed = (a.bits_words + 3) / 4;
    const bool bits_pieces = bits_p != nullptr && (reinterpret_cast<uintptr_t>(a.bits) & 15) == 0 &&
                             a.bits_sw == 1 && a.bits_sr % 4 == 0 && a.bits_sl % 4 == 0 && a.bits_words > 0 &&
                             bits_p->shape[layered_table ? 2 : 1] >= 4 * bits_pieces_needed &&
                             bits_pieces_needed <= static_cast<int64_t>(kPipeBitPieces);
    // Batch and table rows are kept as 32-bit indices (all ones = none).
    // Tables: int16 local slots, or int32 global slots in the single-level form.
    const bool pipe_table = local || (mapping == nullptr && table.dtype == EKV_INT32);
    a.pipe = pipe_table && pieces_layout && dense && a.bits_staged && bits_pieces &&
                     width <= kChunkLanes &&
                     batch > 0 && batch < (int64_t{1} << 31) && a.table_rows > 0 &&
                     a.table_rows < (int64_t{1} << 31) && a.table_cols > 0 && count * layers < (int64_t{1} << 31)
                 ? 1
                 : 0;
    if (check_only()) {
        return 0;
    }
    if (topk.dtype == EKV_INT64) {
        launch_table<int64_t>(a, table.dtype, map_dtype, compact, dense, grid, s);
    } else {
        launch_table<int32_t>(a, table.dtype, map_dtype, compact, dense, grid, s);
    }
    check_hip(hipGetLastError(), "launch resident lookup");
    return 0;
}

// Per-position bitmaps (shift 0) of any layout: a wave turns 64 consecutive
// entries of a row into two words with a ballot, four such groups per
// iteration with their loads in flight together; a wave-stride loop covers
// every (layer, row, 64-entry group).
constexpr int kBitmapGroups = 4;

template <typename TableT>
__global__ __launch_bounds__(kThreads) void residency_bits_kernel(const TableT* __restrict__ table, int64_t t_sl,
                                                                  int64_t t_sr, int64_t t_sc, int64_t rows,
                                                                  int64_t cols, int32_t* __restrict__ bits,
                                                                  int64_t b_sl, int64_t b_sr, int64_t b_sw,
                                                                  int64_t groups_per_row, int64_t total_groups) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = int64_t{gridDim.x} * (kThreads / 64);
    for (int64_t g0 = (int64_t{blockIdx.x} * (kThreads / 64) + (threadIdx.x >> 6)) * kBitmapGroups;
         g0 < total_groups; g0 += waves * kBitmapGroups) {
        bool set[kBitmapGroups];
        int32_t* out[kBitmapGroups];
        int64_t group[kBitmapGroups];
#pragma unroll
        for (int k = 0; k < kBitmapGroups; ++k) {
            const int64_t g = g0 + k;   // uniform over the wave
            const bool live = g < total_groups;
            group[k] = live ? g % groups_per_row : 0;
            const int64_t row_index = live ? g / groups_per_row : 0;   // layer * rows + row
            const int64_t layer = row_index / rows;
            const int64_t row = row_index - layer * rows;
            const int64_t pos = group[k] * 64 + lane;
            set[k] = live && pos < cols && table[layer * t_sl + row * t_sr + pos * t_sc] != 0;
            out[k] = live ? bits + layer * b_sl + row * b_sr : nullptr;
        }
#pragma unroll
        for (int k = 0; k < kBitmapGroups; ++k) {
            const uint64_t mask = __ballot(set[k]);
            const int64_t word = group[k] * 2;
            if (out[k] != nullptr && lane == 0) {
                out[k][word * b_sw] = static_cast<int32_t>(static_cast<uint32_t>(mask));
            } else if (out[k] != nullptr && lane == 1 && group[k] * 64 + 32 < cols) {
                out[k][(word + 1) * b_sw] = static_cast<int32_t>(static_cast<uint32_t>(mask >> 32));
            }
        }
    }
}

// Summary rows (shift > 0) of any layout (strided entries, rows that do not
// come in whole 16-byte pieces): one wave per summary word covers the 32 << shift
// positions of its 32 groups, 64 consecutive entries per iteration, each lane
// OR-ing the bit of its entry's group; the wave's bits are OR-reduced and
// lane 0 writes the word.
template <typename TableT>
__global__ __launch_bounds__(kThreads) void residency_summary_kernel(
    const TableT* __restrict__ table, int64_t t_sl, int64_t t_sr, int64_t t_sc, int64_t rows, int64_t cols,
    int32_t* __restrict__ bits, int64_t b_sl, int64_t b_sr, int64_t b_sw, int64_t words_per_row, int64_t total_words,
    uint32_t shift) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = int64_t{gridDim.x} * (kThreads / 64);
    for (int64_t g = int64_t{blockIdx.x} * (kThreads / 64) + (threadIdx.x >> 6); g < total_words; g += waves) {
        const int64_t word = g % words_per_row;
        const int64_t row_index = g / words_per_row;   // layer * rows + row
        const int64_t layer = row_index / rows;
        const int64_t row = row_index - layer * rows;
        const TableT* entries = table + layer * t_sl + row * t_sr;
        const int64_t first = (word * 32) << shift;
        const int64_t stop = std::min<int64_t>(first + (int64_t{32} << shift), cols);
        uint32_t acc = 0;
        for (int64_t pos = first + lane; pos < stop; pos += 64) {
            acc |= static_cast<uint32_t>(entries[pos * t_sc] != 0) << ((pos >> shift) & 31);
        }
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) {
            acc |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), offset));
        }
        if (lane == 0) {
            bits[layer * b_sl + row * b_sr + word * b_sw] = static_cast<int32_t>(acc);
        }
    }
}

// Nonzero entries of one 16-byte piece of a table row: bit k = entry k.
template <typename TableT>
__device__ inline uint32_t piece_nonzero(const uint4 v) {
    if constexpr (sizeof(TableT) == 2) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t bits = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bits |= static_cast<uint32_t>((w[i] & 0xffffu) != 0) << (2 * i);
            bits |= static_cast<uint32_t>((w[i] >> 16) != 0) << (2 * i + 1);
        }
        return bits;
    } else if constexpr (sizeof(TableT) == 4) {
        return static_cast<uint32_t>(v.x != 0) | (static_cast<uint32_t>(v.y != 0) << 1) |
               (static_cast<uint32_t>(v.z != 0) << 2) | (static_cast<uint32_t>(v.w != 0) << 3);
    } else {
        return static_cast<uint32_t>((v.x | v.y) != 0) | (static_cast<uint32_t>((v.z | v.w) != 0) << 1);
    }
}

// Group bits of a piece's n entry bits: bit i = any of entries
// [i << shift, (i + 1) << shift); one bit when a group spans the piece.
__device__ inline uint32_t fold_groups(uint32_t bits, uint32_t n, uint32_t shift) {
    if ((1u << shift) >= n) {
        return bits != 0 ? 1u : 0u;
    }
    const uint32_t mask = (1u << (1u << shift)) - 1;   // shift <= 2 here: groups of 1, 2 or 4 entries
    uint32_t out = 0;
    for (uint32_t i = 0; i < (n >> shift); ++i) {
        out |= static_cast<uint32_t>(((bits >> (i << shift)) & mask) != 0) << i;
    }
    return out;
}

// Summary words of contiguous rows that come in whole 16-byte pieces (T a
// multiple of 16 / sizeof(entry), 16-byte aligned rows). A word's
// 32 << shift positions are ppw = (32 << shift) / E pieces of E entries; a
// segment of seg = min(ppw, 64) lanes builds it, each lane loading every
// seg-th piece with one 16-byte load and OR-ing that piece's group bits into
// place; shuffles over seg/2, ..., 1 lanes OR the segment and its first lane
// writes the word. A wave takes kSummarySets groups of 64 / seg consecutive words per
// iteration (for ppw <= 64: kSummarySets contiguous KiB, one 1 KiB load instruction
// each, all in flight before any is used) and strides over every summary word
// of every (layer, row).
constexpr int kSummarySets = 4;

template <typename TableT>
__global__ __launch_bounds__(kThreads) void residency_pieces_kernel(
    const TableT* __restrict__ table, int64_t t_sl, int64_t t_sr, FastDiv rows_div, int64_t cols,
    int32_t* __restrict__ bits, int64_t b_sl, int64_t b_sr, int64_t b_sw, FastDiv words_div, uint32_t total_words,
    uint32_t shift, uint32_t seg_log2, uint32_t per_lane) {
    constexpr uint32_t kE = 16 / sizeof(TableT);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t in_seg = lane & ((1u << seg_log2) - 1);
    const uint32_t words_per_wave = 64u >> seg_log2;
    const uint32_t wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const uint32_t step = gridDim.x * (kThreads / 64) * words_per_wave * kSummarySets;
    for (uint32_t first = wave * words_per_wave * kSummarySets; first < total_words; first += step) {
        const TableT* entries[kSummarySets];
        int64_t word_first[kSummarySets], out_at[kSummarySets];
        bool live[kSummarySets];
        uint32_t acc[kSummarySets];
#pragma unroll
        for (int k = 0; k < kSummarySets; ++k) {
            const uint32_t gw = first + k * words_per_wave + (lane >> seg_log2);
            live[k] = gw < total_words;
            const uint32_t row_index = words_div.div(live[k] ? gw : 0);   // layer * rows + row
            const uint32_t word = (live[k] ? gw : 0) - row_index * words_div.divisor;
            const uint32_t layer = rows_div.div(row_index);
            const uint32_t row = row_index - layer * rows_div.divisor;
            entries[k] = table + layer * t_sl + row * t_sr;
            word_first[k] = static_cast<int64_t>(word) << (5 + shift);
            out_at[k] = layer * b_sl + row * b_sr + int64_t{word} * b_sw;
            acc[k] = 0;
        }
        for (uint32_t j = 0; j < per_lane; ++j) {
            const uint32_t piece = in_seg + (j << seg_log2);
            uint4 v[kSummarySets];
            bool in[kSummarySets];
#pragma unroll
            for (int k = 0; k < kSummarySets; ++k) {
                const int64_t pos = word_first[k] + int64_t{piece} * kE;
                in[k] = live[k] && pos < cols;
                v[k] = in[k] ? *reinterpret_cast<const uint4*>(entries[k] + pos) : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int k = 0; k < kSummarySets; ++k) {
                if (in[k]) {
                    acc[k] |= fold_groups(piece_nonzero<TableT>(v[k]), kE, shift) << ((piece * kE) >> shift);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kSummarySets; ++k) {
            for (uint32_t offset = (1u << seg_log2) >> 1; offset > 0; offset >>= 1) {
                acc[k] |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc[k]), static_cast<int>(offset)));
            }
            if (live[k] && in_seg == 0) {
                bits[out_at[k]] = static_cast<int32_t>(acc[k]);
            }
        }
    }
}

template <typename TableT>
void launch_residency_bits(const ekv_tensor& table, const ekv_tensor& bits, int d, int64_t layers, int64_t rows,
                           int64_t cols, int64_t shift, hipStream_t s) {
    const bool layered = table.ndim == 3;
    const int64_t t_sl = layered ? table.stride[0] : 0, b_sl = layered ? bits.stride[0] : 0;
    const auto* entries = static_cast<const TableT*>(table.data);
    auto* out = static_cast<int32_t*>(bits.data);
    const int64_t words_per_row = summary_words(cols, shift);
    const int64_t total = layers * rows * words_per_row;
    constexpr int64_t kE = 16 / static_cast<int64_t>(sizeof(TableT));
    const auto piece_aligned = [](int64_t elements) { return (elements * static_cast<int64_t>(sizeof(TableT))) % 16 == 0; };
    const bool pieces = table.stride[d + 1] == 1 && cols % kE == 0 &&
                        (reinterpret_cast<uintptr_t>(table.data) & 15) == 0 && piece_aligned(table.stride[d]) &&
                        (!layered || piece_aligned(t_sl)) && total < (int64_t{1} << 31);
    if (pieces) {
        const int64_t ppw = (int64_t{32} << shift) / kE;   // pieces per summary word (a power of two >= 2)
        uint32_t seg_log2 = 0;
        while ((int64_t{1} << seg_log2) < std::min<int64_t>(ppw, 64)) {
            ++seg_log2;
        }
        const int64_t per_lane = ppw >> seg_log2;
        const int64_t words_per_block = (kThreads / 64) * (64 >> seg_log2) * kSummarySets;
        const int64_t blocks = std::min<int64_t>((total + words_per_block - 1) / words_per_block, 65536);
        residency_pieces_kernel<TableT><<<dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, s>>>(
            entries, t_sl, table.stride[d], FastDiv(static_cast<uint32_t>(rows)), cols, out, b_sl, bits.stride[d],
            bits.stride[d + 1], FastDiv(static_cast<uint32_t>(words_per_row)), static_cast<uint32_t>(total),
            static_cast<uint32_t>(shift), seg_log2, static_cast<uint32_t>(per_lane));
        return;
    }
    if (shift == 0) {
        const int64_t groups_per_row = (cols + 63) / 64;
        const int64_t groups = layers * rows * groups_per_row;
        const int64_t blocks = std::min<int64_t>((groups + 4 * kBitmapGroups - 1) / (4 * kBitmapGroups), 65536);
        residency_bits_kernel<TableT><<<dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, s>>>(
            entries, t_sl, table.stride[d], table.stride[d + 1], rows, cols, out, b_sl, bits.stride[d],
            bits.stride[d + 1], groups_per_row, groups);
        return;
    }
    const int64_t blocks = std::min<int64_t>((total + 3) / 4, 65536);
    residency_summary_kernel<TableT><<<dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, s>>>(
        entries, t_sl, table.stride[d], table.stride[d + 1], rows, cols, out, b_sl, bits.stride[d],
        bits.stride[d + 1], words_per_row, total, static_cast<uint32_t>(shift));
}

int residency_bits(const ekv_tensor* table_p, const ekv_tensor* bits_p, int64_t shift, void* stream) {
    const ekv_tensor& table = need(table_p, "table");
    const ekv_tensor& bits = need(bits_p, "resident_bits");
    if (table.dtype != EKV_INT16) {
        need_index(table, "table");
    }
    if (table.ndim != 2 && table.ndim != 3) {
        throw std::invalid_argument("table must be [R, T] or [L, R, T]");
    }
    if (bits.dtype != EKV_INT32 || bits.ndim != table.ndim) {
        throw std::invalid_argument("resident_bits must be int32 with the table's number of dimensions");
    }
    if (shift < 0 || shift > kMaxBitsShift) {
        throw std::invalid_argument("bits_shift must be 0.." + std::to_string(kMaxBitsShift));
    }
    const bool layered = table.ndim == 3;
    const int d = layered ? 1 : 0;
    const int64_t layers = layered ? table.shape[0] : 1;
    if (layered) {
        need_dim(bits, 0, layers, "resident_bits");
    }
    need_dim(bits, d, table.shape[d], "resident_bits");
    const int64_t rows = table.shape[d], cols = table.shape[d + 1];
    if (bits.shape[d + 1] < summary_words(cols, shift)) {
        throw std::invalid_argument("resident_bits needs ceil(ceil(T / 2^bits_shift) / 32) words per row");
    }
    if (layers * rows * cols == 0) {
        return 0;
    }
    need_data(table, "table");
    need_data(bits, "resident_bits");
    const auto s = static_cast<hipStream_t>(stream);
    if (table.dtype == EKV_INT64) {
        launch_residency_bits<int64_t>(table, bits, d, layers, rows, cols, shift, s);
    } else if (table.dtype == EKV_INT16) {
        launch_residency_bits<int16_t>(table, bits, d, layers, rows, cols, shift, s);
    } else {
        launch_residency_bits<int32_t>(table, bits, d, layers, rows, cols, shift, s);
    }
    check_hip(hipGetLastError(), "launch residency bits");
    return 0;
}

}  // namespace
}  // namespace ekv

extern "C" int ekv_resolve_resident_bits(const ekv_tensor* topk, const ekv_tensor* table,
                                         const ekv_tensor* resident_bits, int64_t bits_shift,
                                         const ekv_tensor* rows, const ekv_tensor* lengths,
                                         const ekv_tensor* selected, const ekv_tensor* output,
                                         const ekv_tensor* misses, const ekv_tensor* miss_count,
                                         int64_t block_size, void* stream) {
    return ekv::guarded(-1, [&] {
        if (resident_bits == nullptr) {
            throw std::invalid_argument("resident_bits is required");
        }
        return ekv::resolve_resident(topk, table, nullptr, rows, lengths, selected, output, misses, miss_count,
                                     resident_bits, block_size, stream, nullptr, bits_shift);
    });
}

extern "C" int ekv_resolve_resident_local(const ekv_tensor* topk, const ekv_tensor* table,
                                          const ekv_tensor* slot_base, const ekv_tensor* resident_bits,
                                          int64_t bits_shift, const ekv_tensor* rows, const ekv_tensor* lengths,
                                          const ekv_tensor* selected, const ekv_tensor* output,
                                          const ekv_tensor* misses, const ekv_tensor* miss_count,
                                          int64_t block_size, void* stream) {
    return ekv::guarded(-1, [&] {
        if (slot_base == nullptr) {
            throw std::invalid_argument("slot_base is required");
        }
        return ekv::resolve_resident(topk, table, nullptr, rows, lengths, selected, output, misses, miss_count,
                                     resident_bits, block_size, stream, slot_base, bits_shift);
    });
}

extern "C" int ekv_residency_bits(const ekv_tensor* table, const ekv_tensor* resident_bits, int64_t bits_shift,
                                  void* stream) {
    return ekv::guarded(-1, [&] { return ekv::residency_bits(table, resident_bits, bits_shift, stream); });
}

extern "C" int ekv_resolve_resident(const ekv_tensor* topk, const ekv_tensor* table, const ekv_tensor* mapping,
                                    const ekv_tensor* rows, const ekv_tensor* lengths,
                                    const ekv_tensor* selected, const ekv_tensor* output,
                                    const ekv_tensor* misses, const ekv_tensor* miss_count,
                                    int64_t block_size, void* stream) {
    return ekv::guarded(-1, [&] {
        return ekv::resolve_resident(topk, table, mapping, rows, lengths, selected, output, misses, miss_count,
                                     nullptr, block_size, stream);
    });
}

extern "C" int ekv_abi_version(void) { return EKV_ABI_VERSION; }
