// Byte-exact comparison of K/V rows held in two plane sets (gfx950).
//
// Serves the logical-shadow check (bitwise oracle contract of
// adaptive_sparse/logical_shadow.py:45-123): the rows a decode step or a
// migration left in the pool, at their physical slots, are compared with a
// shadow copy at their logical slots. The reference compares int16 views of
// every K and V row (:72-75, :108-123); comparing bytes is the same relation.
//
//   equal[l, b, w] =  1  every kv plane's row a_rows[l, b, w] of set A equals
//                        row b_rows[l, b, w] of set B byte for byte
//                     0  some byte differs
//                    -1  either row index lies outside its planes ([0, rows)):
//                        neither row is read
//
// One wave per (l, b, w) item, grid-stride over items: the lanes read
// VW-byte pieces of both rows of every kv plane, and a ballot decides.
#include "../../include/ekv_kernels.h"
#include "ekv_common.h"
#include "ekv_tensor_util.h"
#include "ekv_vec.h"

#include <algorithm>

namespace ekv {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct CompareArgs {
    const char* a_base;
    int64_t a_layer_stride, a_kv_stride, a_row_stride, a_rows_count;
    const char* b_base;
    int64_t b_layer_stride, b_kv_stride, b_row_stride, b_rows_count;
    int64_t row_bytes, kv;
    const void* a_rows;
    int64_t ar_l, ar_b, ar_w;
    int32_t a64;
    const void* b_rows;
    int64_t br_l, br_b, br_w;
    int32_t b64;
    int32_t* equal;
    int64_t eq_l, eq_b, eq_w;
    int64_t items, B, W;
};

__device__ __forceinline__ int64_t row_index(const void* p, int64_t i, int32_t is64) {
    return is64 ? static_cast<const int64_t*>(p)[i] : static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

template <int VW>
__device__ __forceinline__ bool differs(typename Vec<VW>::type x, typename Vec<VW>::type y) {
    if constexpr (VW == 16) {
        return ((x[0] ^ y[0]) | (x[1] ^ y[1]) | (x[2] ^ y[2]) | (x[3] ^ y[3])) != 0u;
    } else if constexpr (VW == 8) {
        return ((x[0] ^ y[0]) | (x[1] ^ y[1])) != 0u;
    } else {
        return x != y;
    }
}

template <int VW>
__global__ __launch_bounds__(kThreads) void compare_rows_kernel(const CompareArgs a) {
    using V = typename Vec<VW>::type;
    const int lane = threadIdx.x & 63;
    const int64_t stride = int64_t{gridDim.x} * kWaves;
    for (int64_t item = int64_t{blockIdx.x} * kWaves + (threadIdx.x >> 6); item < a.items; item += stride) {
        // Wave-uniform item: every branch below is uniform over the wave.
        const int64_t w = item % a.W;
        const int64_t q = item / a.W;
        const int64_t b = q % a.B;
        const int64_t l = q / a.B;
        const int64_t ra = row_index(a.a_rows, l * a.ar_l + b * a.ar_b + w * a.ar_w, a.a64);
        const int64_t rb = row_index(a.b_rows, l * a.br_l + b * a.br_b + w * a.br_w, a.b64);
        int32_t flag = -1;
        if (ra >= 0 && ra < a.a_rows_count && rb >= 0 && rb < a.b_rows_count) {
            bool differ = false;
            for (int64_t kv = 0; kv < a.kv; ++kv) {
                const char* pa = a.a_base + l * a.a_layer_stride + kv * a.a_kv_stride + ra * a.a_row_stride;
                const char* pb = a.b_base + l * a.b_layer_stride + kv * a.b_kv_stride + rb * a.b_row_stride;
                for (int64_t off = int64_t{lane} * VW; off < a.row_bytes; off += 64 * VW) {
                    const V x = *reinterpret_cast<const V*>(pa + off);
                    const V y = *reinterpret_cast<const V*>(pb + off);
                    differ = differ || differs<VW>(x, y);
                }
            }
            flag = __ballot(differ) != 0 ? 0 : 1;
        }
        if (lane == 0) {
            a.equal[l * a.eq_l + b * a.eq_b + w * a.eq_w] = flag;
        }
    }
}

void need_rows(const ekv_tensor& t, const char* name) {
    need_ndim(t, 3, name);
    need_index(t, name);
}

int compare_kv(const ekv_planes* a, const ekv_tensor* a_rows_p, const ekv_planes* b, const ekv_tensor* b_rows_p,
               const ekv_tensor* equal_p, void* stream) {
    if (a == nullptr || b == nullptr) {
        throw std::invalid_argument("both plane sets are required");
    }
    for (const ekv_planes* p : {a, b}) {
        if (p->layers < 0 || p->rows < 0 || p->row_bytes < 0 || (p->kv != 1 && p->kv != 2)) {
            throw std::invalid_argument("planes: layers/rows/row_bytes must be >= 0 and kv 1 or 2");
        }
    }
    if (a->row_bytes != b->row_bytes || a->kv != b->kv) {
        throw std::invalid_argument("plane sets differ in row bytes or kv");
    }
    const ekv_tensor& a_rows = need(a_rows_p, "a_rows");
    const ekv_tensor& b_rows = need(b_rows_p, "b_rows");
    const ekv_tensor& equal = need(equal_p, "equal");
    need_rows(a_rows, "a_rows");
    need_rows(b_rows, "b_rows");
    need_ndim(equal, 3, "equal");
    if (equal.dtype != EKV_INT32) {
        throw std::invalid_argument("equal must be int32");
    }
    for (int d = 0; d < 3; ++d) {
        need_dim(b_rows, d, a_rows.shape[d], "b_rows");
        need_dim(equal, d, a_rows.shape[d], "equal");
    }
    const int64_t L = a_rows.shape[0], B = a_rows.shape[1], W = a_rows.shape[2];
    if (L > a->layers || L > b->layers) {
        throw std::invalid_argument("row lists name more layers than the planes hold");
    }
    const int64_t items = L * B * W;
    if (items == 0) {
        return 0;
    }
    for (const auto* t : {&a_rows, &b_rows, &equal}) {
        need_data(*t, "row list");
    }
    if ((a->base == nullptr && a->rows > 0) || (b->base == nullptr && b->rows > 0)) {
        throw std::invalid_argument("null plane base");
    }
    CompareArgs args{};
    args.a_base = static_cast<const char*>(a->base);
    args.a_layer_stride = a->layer_stride, args.a_kv_stride = a->kv_stride, args.a_row_stride = a->row_stride;
    args.a_rows_count = a->rows;
    args.b_base = static_cast<const char*>(b->base);
    args.b_layer_stride = b->layer_stride, args.b_kv_stride = b->kv_stride, args.b_row_stride = b->row_stride;
    args.b_rows_count = b->rows;
    args.row_bytes = a->row_bytes;
    args.kv = a->kv;
    args.a_rows = a_rows.data;
    args.ar_l = a_rows.stride[0], args.ar_b = a_rows.stride[1], args.ar_w = a_rows.stride[2];
    args.a64 = a_rows.dtype == EKV_INT64;
    args.b_rows = b_rows.data;
    args.br_l = b_rows.stride[0], args.br_b = b_rows.stride[1], args.br_w = b_rows.stride[2];
    args.b64 = b_rows.dtype == EKV_INT64;
    args.equal = static_cast<int32_t*>(equal.data);
    args.eq_l = equal.stride[0], args.eq_b = equal.stride[1], args.eq_w = equal.stride[2];
    args.items = items;
    args.B = B;
    args.W = W;
    const int vw = pick_vector_width({a->row_bytes, reinterpret_cast<int64_t>(a->base), a->layer_stride,
                                      a->kv_stride, a->row_stride, reinterpret_cast<int64_t>(b->base),
                                      b->layer_stride, b->kv_stride, b->row_stride});
    const int64_t groups = std::min<int64_t>((items + kWaves - 1) / kWaves, int64_t{1} << 20);
    const dim3 grid(static_cast<uint32_t>(groups)), block(kThreads);
    const auto s = static_cast<hipStream_t>(stream);
    switch (vw) {
        case 16: compare_rows_kernel<16><<<grid, block, 0, s>>>(args); break;
        case 8: compare_rows_kernel<8><<<grid, block, 0, s>>>(args); break;
        case 4: compare_rows_kernel<4><<<grid, block, 0, s>>>(args); break;
        case 2: compare_rows_kernel<2><<<grid, block, 0, s>>>(args); break;
        default: compare_rows_kernel<1><<<grid, block, 0, s>>>(args); break;
    }
    check_hip(hipGetLastError(), "launch row comparison");
    return 0;
}

}  // namespace
}  // namespace ekv

extern "C" int ekv_compare_kv(const ekv_planes* a, const ekv_tensor* a_rows, const ekv_planes* b,
                              const ekv_tensor* b_rows, const ekv_tensor* equal, void* stream) {
    return ekv::guarded(-1, [&] { return ekv::compare_kv(a, a_rows, b, b_rows, equal, stream); });
}
