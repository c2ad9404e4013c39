// Row-copy engine for the sparse KV gather family (gfx950).
//
// Every operation here moves whole rows of bytes: a row's source and
// destination addresses come from an address mode (below), then the bytes
// are copied with VW-byte lane accesses (16 B = one global_load_dwordx4 per
// lane whenever alignment allows).
//
// Small rows (row_bytes <= one tile of 256 lanes x kUnroll x VW bytes): a
// workgroup takes a tile of whole rows. Phase 1: one thread per row computes
// (source, destination) byte offsets into LDS. Phase 2: the tile's vectors are
// spread over the 256 lanes, each lane issuing kUnroll independent loads
// before its kUnroll stores, so a 512 B K/V row is 32 lanes and a wave moves
// two rows per instruction. Large rows are cut into tile-sized segments, one
// segment per workgroup iteration. Destinations are written with non-temporal
// stores: gathered rows are consumed by the next kernel, not re-read here.
//
// Address modes:
//   KvGather / KvScatter  - planes (layer, kv) x slot rows <-> dense rows
//                           (l, b, kv, k); slots outside [zero_below, rows)
//                           give zero rows (gather) or are skipped (scatter).
//   RowsDirect / RowsIndirect - experimental/sparse_read.py:11-30 semantics
//                           over one flat payload tensor.
#include "../../include/ekv_kernels.h"
#include "ekv_common.h"
#include "ekv_device.h"
#include "ekv_fastdiv.h"
#include "ekv_tensor_util.h"
#include "ekv_vec.h"

#include <algorithm>
#include <stdexcept>
#include <atomic>
#include <type_traits>

namespace ekv {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;  // independent VW-byte loads in flight per lane
// KV gathers of small rows reserve LDS they do not use, so that at most 3 of
// their workgroups share a CU (160 KiB of LDS per CU on MI355X; 4 KiB static
// + 48 KiB reserved per workgroup). Fewer gathers in flight per CU measured
// faster on the decode shapes: 5 per CU (the register limit) 5.08 ms, 4 per
// CU 5.01 ms, 3 per CU 4.91 ms, 2 per CU 5.06 ms for 31.5 M rows of 512 B.
// (Large rows, and the lookup kernels, measured no gain from fewer groups.)
constexpr size_t kGatherLdsReserve = 49152;
// MI355X has 8 XCDs; workgroups are dispatched to them round robin. Dealing
// each XCD one contiguous range of tiles keeps neighbouring rows (same
// request region of a plane, adjacent slot reads) on one XCD's L2 and TLBs:
// +13 % on the 60-layer decode gather compared with plain tile order.
constexpr int64_t kXcdCount = 8;

enum Mode : int {
    KvGather = 0, KvScatter = 1, RowsDirect = 2, RowsIndirect = 3, KvGather64 = 4, KvScatter64 = 5, KvMove = 6
};

constexpr bool is_kv_mode(int m) { return m == KvGather || m == KvScatter || m == KvGather64 || m == KvScatter64; }
constexpr bool is_gather_mode(int m) { return m == KvGather || m == KvGather64; }

struct EngineArgs {
    // Byte bases: the engine copies from src_base + src_off to dst_base + dst_off.
    const char* src_base;
    char* dst_base;
    int64_t units;           // rows in the job
    int64_t row_bytes;
    // Small-row tiling.
    uint32_t rows_per_tile;
    uint32_t vecs_per_row;
    FastDiv vec_div;
    // Large-row segmentation.
    int64_t seg_bytes;
    int64_t segs_per_row;
    int64_t tiles;           // work items of the grid-stride loop
    uint32_t xcd_groups;     // 0: no remap; else tiles are dealt in XCD-contiguous ranges

    // Kv modes: unit u = ((l * B + b) * KV + kv) * K + k.
    char* pool;
    int64_t layer_stride, kv_stride, row_stride, pool_rows;
    char* dense;
    int64_t d_sl, d_sb, d_skv, d_sk;
    const void* slots;
    int64_t s_sl, s_sb, s_sk;
    int32_t slots64;
    int64_t zero_below;
    int64_t K, KV, B;
    FastDiv div_k, div_kv, div_b;
    bool small_units;        // units < 2^31: decompose with FastDiv

    // Move mode: rows src_rows[l, b, i] of the source planes -> rows
    // dst_rows[l, b, i] of the destination planes, for i < counts[l, b].
    const char* msrc;
    int64_t ms_layer_stride, ms_kv_stride, ms_row_stride, ms_rows;
    const int32_t* move_src_rows;
    int64_t msr_l, msr_b, msr_i;
    const int32_t* move_dst_rows;
    int64_t mdr_l, mdr_b, mdr_i;
    const int32_t* move_counts;
    int64_t mc_l, mc_b;

    // Rows modes: unit u = b * S + s.
    const char* raw;
    int64_t raw_elems, itemsize, width, request_stride, sink;
    IndexRef positions_b;    // positions stride over b (dim 0)
    int64_t pos_ss;          // positions stride over s (dim 1)
    IndexRef request_ids, lengths;
    const void* request_table;
    int64_t rt_sr, rt_sc, rt_rows, rt_cols;
    int32_t rt64;
    IndexRef slot_offsets;
    int64_t slot_len;
    int64_t out_sb, out_ss;  // output strides in bytes
    int64_t S;
};

// (source offset, destination offset) in bytes of one row; -1 source means a
// zero row, -1 destination means the row is not written.
__device__ __forceinline__ void split_unit(const EngineArgs& a, int64_t u, int64_t& l, int64_t& b, int64_t& kv,
                                           int64_t& k) {
    if (a.small_units) {
        const uint32_t u32 = static_cast<uint32_t>(u);
        const uint32_t q1 = a.div_k.div(u32);
        k = u32 - q1 * static_cast<uint32_t>(a.K);
        const uint32_t q2 = a.div_kv.div(q1);
        kv = q1 - q2 * static_cast<uint32_t>(a.KV);
        const uint32_t q3 = a.div_b.div(q2);
        b = q2 - q3 * static_cast<uint32_t>(a.B);
        l = q3;
    } else {
        k = u % a.K;
        int64_t q = u / a.K;
        kv = q % a.KV;
        q /= a.KV;
        b = q % a.B;
        l = q / a.B;
    }
}

template <int M>
__device__ __forceinline__ void locate(const EngineArgs& a, int64_t u, int64_t& src, int64_t& dst) {
    if constexpr (M == KvMove) {
        int64_t l, b, kv, k;
        split_unit(a, u, l, b, kv, k);
        src = -1;
        dst = -1;
        if (k < a.move_counts[l * a.mc_l + b * a.mc_b]) {
            const int64_t from = a.move_src_rows[l * a.msr_l + b * a.msr_b + k * a.msr_i];
            const int64_t to = a.move_dst_rows[l * a.mdr_l + b * a.mdr_b + k * a.mdr_i];
            if (from >= 0 && from < a.ms_rows && to >= a.zero_below && to < a.pool_rows) {
                src = l * a.ms_layer_stride + kv * a.ms_kv_stride + from * a.ms_row_stride;
                dst = l * a.layer_stride + kv * a.kv_stride + to * a.row_stride;
            }
        }
    } else if constexpr (is_kv_mode(M)) {
        using SlotT = typename std::conditional<(M == KvGather64 || M == KvScatter64), int64_t, int32_t>::type;
        int64_t k, kv, b, l;
        split_unit(a, u, l, b, kv, k);
        const int64_t slot = static_cast<const SlotT*>(a.slots)[l * a.s_sl + b * a.s_sb + k * a.s_sk];
        const bool valid = slot >= a.zero_below && slot < a.pool_rows;
        const int64_t pool_off = l * a.layer_stride + kv * a.kv_stride + slot * a.row_stride;
        const int64_t dense_off = l * a.d_sl + b * a.d_sb + kv * a.d_skv + k * a.d_sk;
        if constexpr (is_gather_mode(M)) {
            src = valid ? pool_off : -1;
            dst = dense_off;
        } else {
            src = dense_off;
            dst = valid ? pool_off : -1;
        }
    } else {
        const int64_t b = u / a.S;
        const int64_t s = u - b * a.S;
        const int64_t position = load_index(a.positions_b.data, a.positions_b.is64,
                                            b * a.positions_b.stride + s * a.pos_ss);
        const int64_t req = a.request_ids[b];
        const int64_t length = a.lengths[b];
        const bool valid = position >= 0 && position < length;
        int64_t element = -1;
        if (valid) {
            if constexpr (M == RowsDirect) {
                element = a.sink + req * a.request_stride + position * a.width;
            } else {
                if (req >= 0 && req < a.rt_rows && position < a.rt_cols) {
                    const int64_t logical =
                        load_index(a.request_table, a.rt64, req * a.rt_sr + position * a.rt_sc);
                    if (logical >= 0 && logical < a.slot_len) {
                        element = a.slot_offsets[logical];
                    }
                }
            }
        }
        const bool in_range = element >= 0 && element + a.width <= a.raw_elems;
        src = in_range ? element * a.itemsize : -1;
        dst = b * a.out_sb + s * a.out_ss;
    }
}

// Loads are plain (cached) and stores non-temporal: the copied rows are not
// read again by this kernel, and streaming them past the caches keeps the
// L2 for the row offsets and the source rows.
template <int VW>
__device__ __forceinline__ typename Vec<VW>::type load_vec(const char* p, bool aligned) {
    using V = typename Vec<VW>::type;
    if (aligned) {
        return *reinterpret_cast<const V*>(p);
    }
    V v;
    __builtin_memcpy(&v, p, VW);
    return v;
}

template <int VW>
__device__ __forceinline__ void store_vec(char* p, typename Vec<VW>::type v) {
    using V = typename Vec<VW>::type;
    __builtin_nontemporal_store(v, reinterpret_cast<V*>(p));
}

__device__ __forceinline__ int64_t tile_of(const EngineArgs& a, int64_t iteration_tile) {
    if (a.xcd_groups == 0) {
        return iteration_tile;
    }
    // Consecutive workgroup ids land on different XCDs (round robin); deal
    // each XCD one contiguous range of tiles instead.
    const int64_t per = (a.tiles + a.xcd_groups - 1) / a.xcd_groups;
    const int64_t group = iteration_tile % a.xcd_groups;
    const int64_t index = iteration_tile / a.xcd_groups;
    return group * per + index;
}

template <int M, int VW>
__global__ __launch_bounds__(kThreads) void copy_small_rows(const EngineArgs a) {
    using V = typename Vec<VW>::type;
    constexpr bool kCheckAlign = (M == RowsIndirect) && VW > 1;
    __shared__ int64_t src_off[kThreads];
    __shared__ int64_t dst_off[kThreads];
    const int64_t grid_tiles = (a.xcd_groups == 0) ? a.tiles
                                                    : ((a.tiles + a.xcd_groups - 1) / a.xcd_groups) * a.xcd_groups;
    for (int64_t iteration = blockIdx.x; iteration < grid_tiles; iteration += gridDim.x) {
        const int64_t tile = tile_of(a, iteration);
        if (tile >= a.tiles) {
            continue;  // uniform over the workgroup
        }
        const int64_t first = tile * a.rows_per_tile;
        const int64_t left = a.units - first;
        const uint32_t rows_here = left < a.rows_per_tile ? static_cast<uint32_t>(left) : a.rows_per_tile;
        if (threadIdx.x < rows_here) {
            int64_t s, d;
            locate<M>(a, first + threadIdx.x, s, d);
            src_off[threadIdx.x] = s;
            dst_off[threadIdx.x] = d;
        }
        __syncthreads();
        const uint32_t tile_vecs = rows_here * a.vecs_per_row;
        for (uint32_t base = threadIdx.x; base < tile_vecs; base += kThreads * kUnroll) {
            V v[kUnroll];
            int64_t d[kUnroll];
#pragma unroll
            for (int i = 0; i < kUnroll; ++i) {
                const uint32_t idx = base + i * kThreads;
                d[i] = -1;
                v[i] = V{};
                if (idx < tile_vecs) {
                    const uint32_t r = a.vec_div.div(idx);
                    const uint32_t c = idx - r * a.vecs_per_row;
                    const int64_t s = src_off[r];
                    const int64_t t = dst_off[r];
                    if (t >= 0) {
                        d[i] = t + static_cast<int64_t>(c) * VW;
                        if (s >= 0) {
                            const bool aligned = !kCheckAlign || (s % VW) == 0;
                            v[i] = load_vec<VW>(a.src_base + s + static_cast<int64_t>(c) * VW, aligned);
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kUnroll; ++i) {
                if (d[i] >= 0) {
                    store_vec<VW>(a.dst_base + d[i], v[i]);
                }
            }
        }
        __syncthreads();  // LDS offsets are rewritten by the next tile
    }
}

template <int M, int VW>
__global__ __launch_bounds__(kThreads) void copy_large_rows(const EngineArgs a) {
    using V = typename Vec<VW>::type;
    constexpr bool kCheckAlign = (M == RowsIndirect) && VW > 1;
    for (int64_t item = blockIdx.x; item < a.tiles; item += gridDim.x) {
        const int64_t row = item / a.segs_per_row;
        const int64_t seg = item - row * a.segs_per_row;
        int64_t s, t;
        locate<M>(a, row, s, t);  // uniform over the workgroup
        if (t < 0) {
            continue;
        }
        const int64_t seg_start = seg * a.seg_bytes;
        const int64_t seg_len = std::min<int64_t>(a.seg_bytes, a.row_bytes - seg_start);
        const uint32_t vecs = static_cast<uint32_t>(seg_len / VW);
        const bool aligned = !kCheckAlign || (s % VW) == 0;
        for (uint32_t base = threadIdx.x; base < vecs; base += kThreads * kUnroll) {
            V v[kUnroll];
#pragma unroll
            for (int i = 0; i < kUnroll; ++i) {
                const uint32_t idx = base + i * kThreads;
                v[i] = V{};
                if (idx < vecs && s >= 0) {
                    v[i] = load_vec<VW>(a.src_base + s + seg_start + static_cast<int64_t>(idx) * VW, aligned);
                }
            }
#pragma unroll
            for (int i = 0; i < kUnroll; ++i) {
                const uint32_t idx = base + i * kThreads;
                if (idx < vecs) {
                    store_vec<VW>(a.dst_base + t + seg_start + static_cast<int64_t>(idx) * VW, v[i]);
                }
            }
        }
    }
}

// Compute units of the current device (cached per device).
int64_t device_cus() {
    static std::atomic<int> cached[64];
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    if (device < 0 || device >= 64) {
        throw std::runtime_error("device ordinal out of range");
    }
    int cus = cached[device].load(std::memory_order_relaxed);
    if (cus == 0) {
        check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                  "hipDeviceGetAttribute");
        cus = std::max(1, cus);
        cached[device].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

// A small job (a few thousand rows: one layer of a small batch, a short
// gather) would fill only a fraction of the CUs with full tiles and take one
// tile's latency on each; below this many workgroups per CU its tiles shrink
// so that the grid reaches it (a tile keeps at least one row).
constexpr int64_t kSmallJobGroupsPerCu = 2;

template <int M, int VW>
void launch_engine(EngineArgs a, hipStream_t stream) {
    const int64_t tile_bytes = int64_t{kThreads} * kUnroll * VW;
    const bool small = a.row_bytes <= tile_bytes;
    if (small) {
        a.vecs_per_row = static_cast<uint32_t>(a.row_bytes / VW);
        a.rows_per_tile = static_cast<uint32_t>(std::min<int64_t>(kThreads, tile_bytes / a.row_bytes));
        a.vec_div = FastDiv(a.vecs_per_row);
        a.tiles = (a.units + a.rows_per_tile - 1) / a.rows_per_tile;
        const int64_t wanted = kSmallJobGroupsPerCu * device_cus();
        if (a.tiles < wanted) {
            a.rows_per_tile = static_cast<uint32_t>(std::max<int64_t>(1, (a.units + wanted - 1) / wanted));
            a.tiles = (a.units + a.rows_per_tile - 1) / a.rows_per_tile;
        }
    } else {
        a.seg_bytes = tile_bytes;
        a.segs_per_row = (a.row_bytes + tile_bytes - 1) / tile_bytes;
        a.tiles = a.units * a.segs_per_row;
    }
    // One workgroup per tile; small-row tiles are dealt to the XCDs in contiguous ranges.
    a.xcd_groups = small ? static_cast<uint32_t>(kXcdCount) : 0u;
    const int64_t grid = std::min<int64_t>(a.tiles, 0x7fffffff);
    if (grid <= 0) {
        return;
    }
    if (small) {
        copy_small_rows<M, VW><<<dim3(static_cast<uint32_t>(grid)), dim3(kThreads),
                                 is_gather_mode(M) ? kGatherLdsReserve : 0, stream>>>(a);
    } else {
        copy_large_rows<M, VW><<<dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, stream>>>(a);
    }
}

template <int M>
void launch_vw(const EngineArgs& a, int vw, hipStream_t stream) {
    switch (vw) {
        case 16: launch_engine<M, 16>(a, stream); break;
        case 8: launch_engine<M, 8>(a, stream); break;
        case 4: launch_engine<M, 4>(a, stream); break;
        case 2: launch_engine<M, 2>(a, stream); break;
        default: launch_engine<M, 1>(a, stream); break;
    }
}

void need_planes(const ekv_planes* p) {
    if (p == nullptr) {
        throw std::invalid_argument("planes are required");
    }
    if (p->layers < 0 || p->rows < 0 || p->row_bytes < 0 || (p->kv != 1 && p->kv != 2)) {
        throw std::invalid_argument("planes: layers/rows/row_bytes must be >= 0 and kv 1 or 2");
    }
    if (p->row_bytes > p->row_stride && p->rows > 1) {
        throw std::invalid_argument("planes: row_bytes exceeds row_stride");
    }
}

int kv_copy(bool gather, const ekv_planes* planes, const ekv_tensor* slots_p, const ekv_kv_rows* dense,
            int64_t zero_below, void* stream) {
    need_planes(planes);
    const ekv_tensor& slots = need(slots_p, "slots");
    need_ndim(slots, 3, "slots");
    need_index(slots, "slots");
    if (dense == nullptr) {
        throw std::invalid_argument("dense rows are required");
    }
    const int64_t L = slots.shape[0], B = slots.shape[1], K = slots.shape[2];
    if (zero_below < 0) {
        throw std::invalid_argument("zero_below must be >= 0 (negative slots never address the pool)");
    }
    if (L > planes->layers) {
        throw std::invalid_argument("slots name more layers than the pool holds");
    }
    const int64_t units = L * B * planes->kv * K;
    if (units == 0 || planes->row_bytes == 0) {
        return 0;
    }
    if (planes->base == nullptr || dense->data == nullptr || slots.data == nullptr) {
        throw std::invalid_argument("null pool, dense or slot pointer");
    }
    EngineArgs a{};
    a.units = units;
    a.row_bytes = planes->row_bytes;
    a.pool = static_cast<char*>(planes->base);
    a.layer_stride = planes->layer_stride;
    a.kv_stride = planes->kv_stride;
    a.row_stride = planes->row_stride;
    a.pool_rows = planes->rows;
    a.dense = static_cast<char*>(dense->data);
    a.d_sl = dense->layer_stride;
    a.d_sb = dense->batch_stride;
    a.d_skv = dense->kv_stride;
    a.d_sk = dense->lane_stride;
    a.slots = slots.data;
    a.s_sl = slots.stride[0];
    a.s_sb = slots.stride[1];
    a.s_sk = slots.stride[2];
    a.slots64 = slots.dtype == EKV_INT64;
    a.zero_below = zero_below;
    a.K = K;
    a.KV = planes->kv;
    a.B = B;
    a.small_units = units < (int64_t{1} << 31);
    if (a.small_units) {
        a.div_k = FastDiv(static_cast<uint32_t>(K));
        a.div_kv = FastDiv(static_cast<uint32_t>(planes->kv));
        a.div_b = FastDiv(static_cast<uint32_t>(B));
    }
    a.src_base = gather ? a.pool : a.dense;
    a.dst_base = gather ? a.dense : a.pool;
    const int vw = pick_vector_width({planes->row_bytes, reinterpret_cast<int64_t>(planes->base),
                                      planes->layer_stride, planes->kv_stride, planes->row_stride,
                                      reinterpret_cast<int64_t>(dense->data), dense->layer_stride,
                                      dense->batch_stride, dense->kv_stride, dense->lane_stride});
    if (check_only()) {
        return 0;
    }
    const auto s = static_cast<hipStream_t>(stream);
    if (gather) {
        a.slots64 ? launch_vw<KvGather64>(a, vw, s) : launch_vw<KvGather>(a, vw, s);
    } else {
        a.slots64 ? launch_vw<KvScatter64>(a, vw, s) : launch_vw<KvScatter>(a, vw, s);
    }
    check_hip(hipGetLastError(), gather ? "launch KV gather" : "launch KV scatter");
    return 0;
}

int gather_rows(const ekv_tensor* raw_p, const ekv_tensor* positions_p, const ekv_tensor* request_ids_p,
                const ekv_tensor* lengths_p, const ekv_tensor* request_table_p, const ekv_tensor* slot_offsets_p,
                const ekv_tensor* output_p, int64_t request_stride, int64_t sink_elements, int indirect,
                void* stream) {
    const ekv_tensor& raw = need(raw_p, "raw");
    const ekv_tensor& positions = need(positions_p, "positions");
    const ekv_tensor& request_ids = need(request_ids_p, "request_ids");
    const ekv_tensor& lengths = need(lengths_p, "lengths");
    const ekv_tensor& output = need(output_p, "output");
    need_ndim(raw, 1, "raw");
    need_ndim(positions, 2, "positions");
    need_index(positions, "positions");
    need_ndim(output, 3, "output");
    const int64_t B = positions.shape[0], S = positions.shape[1];
    need_dim(output, 0, B, "output");
    need_dim(output, 1, S, "output");
    const int64_t width = output.shape[2];
    if (output.dtype != raw.dtype) {
        throw std::invalid_argument("output dtype must match raw");
    }
    if (raw.stride[0] != 1 || (width > 1 && output.stride[2] != 1)) {
        throw std::invalid_argument("raw and the rows of output must be contiguous");
    }
    need_ndim(request_ids, 1, "request_ids");
    need_ndim(lengths, 1, "lengths");
    need_index(request_ids, "request_ids");
    need_index(lengths, "lengths");
    need_dim(request_ids, 0, B, "request_ids");
    need_dim(lengths, 0, B, "lengths");
    if (B == 0 || S == 0 || width == 0) {
        return 0;
    }
    const int64_t item = itemsize(raw.dtype);
    EngineArgs a{};
    a.units = B * S;
    a.row_bytes = width * item;
    a.raw = static_cast<const char*>(raw.data);
    a.raw_elems = raw.shape[0];
    a.itemsize = item;
    a.width = width;
    a.request_stride = request_stride;
    a.sink = sink_elements;
    a.positions_b = index_ref(positions, 0);
    a.pos_ss = positions.stride[1];
    a.request_ids = index_ref(request_ids, 0);
    a.lengths = index_ref(lengths, 0);
    a.out_sb = output.stride[0] * item;
    a.out_ss = output.stride[1] * item;
    a.S = S;
    if (indirect) {
        const ekv_tensor& table = need(request_table_p, "request_table");
        const ekv_tensor& offsets = need(slot_offsets_p, "slot_offsets");
        need_ndim(table, 2, "request_table");
        need_index(table, "request_table");
        need_ndim(offsets, 1, "slot_offsets");
        need_index(offsets, "slot_offsets");
        need_data(table, "request_table");
        need_data(offsets, "slot_offsets");
        a.request_table = table.data;
        a.rt_sr = table.stride[0];
        a.rt_sc = table.stride[1];
        a.rt_rows = table.shape[0];
        a.rt_cols = table.shape[1];
        a.rt64 = table.dtype == EKV_INT64;
        a.slot_offsets = index_ref(offsets, 0);
        a.slot_len = offsets.shape[0];
    }
    for (const auto* one : {&raw, &positions, &request_ids, &lengths, &output}) {
        need_data(*one, "tensor");
    }
    a.src_base = a.raw;
    a.dst_base = static_cast<char*>(output.data);
    int vw = pick_vector_width({a.row_bytes, reinterpret_cast<int64_t>(raw.data),
                                reinterpret_cast<int64_t>(output.data), a.out_sb, a.out_ss});
    if (!indirect) {
        vw = std::min(vw, pick_vector_width({sink_elements * item, request_stride * item, width * item}));
    }
    const auto s = static_cast<hipStream_t>(stream);
    if (indirect) {
        launch_vw<RowsIndirect>(a, vw, s);
    } else {
        launch_vw<RowsDirect>(a, vw, s);
    }
    check_hip(hipGetLastError(), "launch row gather");
    return 0;
}

int move_kv(const ekv_planes* src, const ekv_tensor* src_rows_p, const ekv_planes* dst,
            const ekv_tensor* dst_rows_p, const ekv_tensor* counts_p, int64_t zero_below, void* stream) {
    need_planes(src);
    need_planes(dst);
    const ekv_tensor& src_rows = need(src_rows_p, "src_rows");
    const ekv_tensor& dst_rows = need(dst_rows_p, "dst_rows");
    const ekv_tensor& counts = need(counts_p, "counts");
    need_ndim(src_rows, 3, "src_rows");
    need_ndim(dst_rows, 3, "dst_rows");
    need_ndim(counts, 2, "counts");
    for (const auto* t : {&src_rows, &dst_rows, &counts}) {
        if (t->dtype != EKV_INT32) {
            throw std::invalid_argument("move lists and counts must be int32");
        }
    }
    const int64_t L = src_rows.shape[0], B = src_rows.shape[1], K = src_rows.shape[2];
    for (int d = 0; d < 3; ++d) {
        need_dim(dst_rows, d, src_rows.shape[d], "dst_rows");
    }
    need_dim(counts, 0, L, "counts");
    need_dim(counts, 1, B, "counts");
    if (src->row_bytes != dst->row_bytes || src->kv != dst->kv) {
        throw std::invalid_argument("source and destination planes differ in row bytes or kv");
    }
    if (L > src->layers || L > dst->layers) {
        throw std::invalid_argument("move lists name more layers than the planes hold");
    }
    if (zero_below < 0) {
        throw std::invalid_argument("zero_below must be >= 0");
    }
    const int64_t units = L * B * dst->kv * K;
    if (units == 0 || dst->row_bytes == 0) {
        return 0;
    }
    if (src->base == nullptr || dst->base == nullptr) {
        throw std::invalid_argument("null plane base");
    }
    for (const auto* t : {&src_rows, &dst_rows, &counts}) {
        need_data(*t, "move list");
    }
    EngineArgs a{};
    a.units = units;
    a.row_bytes = dst->row_bytes;
    a.layer_stride = dst->layer_stride;
    a.kv_stride = dst->kv_stride;
    a.row_stride = dst->row_stride;
    a.pool_rows = dst->rows;
    a.zero_below = zero_below;
    a.msrc = static_cast<const char*>(src->base);
    a.ms_layer_stride = src->layer_stride;
    a.ms_kv_stride = src->kv_stride;
    a.ms_row_stride = src->row_stride;
    a.ms_rows = src->rows;
    a.move_src_rows = static_cast<const int32_t*>(src_rows.data);
    a.msr_l = src_rows.stride[0], a.msr_b = src_rows.stride[1], a.msr_i = src_rows.stride[2];
    a.move_dst_rows = static_cast<const int32_t*>(dst_rows.data);
    a.mdr_l = dst_rows.stride[0], a.mdr_b = dst_rows.stride[1], a.mdr_i = dst_rows.stride[2];
    a.move_counts = static_cast<const int32_t*>(counts.data);
    a.mc_l = counts.stride[0], a.mc_b = counts.stride[1];
    a.K = K;
    a.KV = dst->kv;
    a.B = B;
    a.small_units = units < (int64_t{1} << 31);
    if (a.small_units) {
        a.div_k = FastDiv(static_cast<uint32_t>(K));
        a.div_kv = FastDiv(static_cast<uint32_t>(dst->kv));
        a.div_b = FastDiv(static_cast<uint32_t>(B));
    }
    a.src_base = a.msrc;
    a.dst_base = static_cast<char*>(dst->base);
    const int vw = pick_vector_width({dst->row_bytes, reinterpret_cast<int64_t>(src->base), src->layer_stride,
                                      src->kv_stride, src->row_stride, reinterpret_cast<int64_t>(dst->base),
                                      dst->layer_stride, dst->kv_stride, dst->row_stride});
    if (check_only()) {
        return 0;
    }
    launch_vw<KvMove>(a, vw, static_cast<hipStream_t>(stream));
    check_hip(hipGetLastError(), "launch KV move");
    return 0;
}

// Pinned host memory that kernels can read and write directly.
int host_alloc(uint64_t bytes, void** host, void** device) {
    if (host == nullptr || device == nullptr || bytes == 0) {
        throw std::invalid_argument("host_alloc needs a positive size and two out pointers");
    }
    *host = nullptr;
    *device = nullptr;
    void* memory = nullptr;
    check_hip(hipHostMalloc(&memory, bytes, hipHostMallocDefault), "hipHostMalloc");
    void* mapped = nullptr;
    const hipError_t status = hipHostGetDevicePointer(&mapped, memory, 0);
    if (status != hipSuccess || mapped == nullptr) {
        (void)hipHostFree(memory);
        fail_hip(status == hipSuccess ? hipErrorInvalidValue : status, "hipHostGetDevicePointer");
    }
    *host = memory;
    *device = mapped;
    return 0;
}

}  // namespace
}  // namespace ekv

extern "C" int ekv_move_kv(const ekv_planes* src, const ekv_tensor* src_rows, const ekv_planes* dst,
                           const ekv_tensor* dst_rows, const ekv_tensor* counts, int64_t zero_below, void* stream) {
    return ekv::guarded(-1, [&] { return ekv::move_kv(src, src_rows, dst, dst_rows, counts, zero_below, stream); });
}

extern "C" int ekv_host_alloc(uint64_t bytes, void** host, void** device) {
    return ekv::guarded(-1, [&] { return ekv::host_alloc(bytes, host, device); });
}

extern "C" int ekv_host_free(void* host) {
    return ekv::guarded(-1, [&] {
        if (host != nullptr) {
            ekv::check_hip(hipHostFree(host), "hipHostFree");
        }
        return 0;
    });
}

extern "C" int ekv_gather_kv(const ekv_planes* planes, const ekv_tensor* slots, const ekv_kv_rows* out,
                             int64_t zero_below, void* stream) {
    return ekv::guarded(-1, [&] { return ekv::kv_copy(true, planes, slots, out, zero_below, stream); });
}

extern "C" int ekv_scatter_kv(const ekv_planes* planes, const ekv_tensor* slots, const ekv_kv_rows* src,
                              int64_t zero_below, void* stream) {
    return ekv::guarded(-1, [&] { return ekv::kv_copy(false, planes, slots, src, zero_below, stream); });
}

extern "C" int ekv_gather_rows(const ekv_tensor* raw, const ekv_tensor* positions, const ekv_tensor* request_ids,
                               const ekv_tensor* lengths, const ekv_tensor* request_table,
                               const ekv_tensor* slot_offsets, const ekv_tensor* output, int64_t request_stride,
                               int64_t sink_elements, int indirect, void* stream) {
    return ekv::guarded(-1, [&] {
        return ekv::gather_rows(raw, positions, request_ids, lengths, request_table, slot_offsets, output,
                                request_stride, sink_elements, indirect, stream);
    });
}
