/*
 * ekv_oracle.c - CPU restatement of the sparse-KV residency hot path.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, the smoke entry point and the bench's
 * CPU-baseline leg call it to verify (and, for the baseline, to time) the
 * HIP kernels. No product code path may call it.
 *
 * Plain scalar C, one element at a time, written to follow the reference's
 * semantics literally rather than to be fast. All index arrays are dense
 * int64 (the Python wrapper converts); payload arrays are raw bytes.
 *
 * Pinned by tests/test_oracle.py against the reference's own known answers
 * (tests/smoke_resident_lookup.py:8-23, tests/bench_resident_lookup.py:38-42,
 * scripts/bench_virtual_addressing.py:47-88), against the independent numpy
 * restatement in oracle/oracle.py, and against brute-force Python loops.
 */
#include <stdint.h>
#include <string.h>

/*
 * Resident lookup. Follows adaptive_sparse/resident_lookup.py:14-26 (Triton)
 * == adaptive_sparse/request_residency.py:819-825 (torch), per lane:
 *   block = topk[l, row, o / bs]; pos = block * bs + o % bs
 *   valid = block >= 0 && pos < lengths[row]
 *   out   = valid ? int32(mapping[table[rows[row], pos]]) : -1
 * Extensions beyond the reference: layer dimension L (table / mapping optionally
 * per layer), mapping == NULL (single level), bounds-guarded lanes -> -1
 * (where the reference would read out of bounds), and the miss list: lanes
 * with valid && out == 0 in ascending order (== torch.nonzero row-major),
 * count in counts[l, row]. Rows not in `selected` are not written.
 */
void oracle_resolve_resident(int64_t L, int64_t B, int64_t K, int64_t bs, const int64_t* topk,
                             const int64_t* table, int table_layered, int64_t R, int64_t T,
                             const int64_t* mapping, int map_layered, int64_t N, const int64_t* rows,
                             const int64_t* lengths, const int64_t* selected, int64_t S, int32_t* output,
                             int32_t* misses, int32_t* counts) {
    const int64_t W = K * bs;
    for (int64_t l = 0; l < L; ++l) {
        for (int64_t i = 0; i < S; ++i) {
            const int64_t row = selected[i];
            if (row < 0 || row >= B) {
                continue;
            }
            const int64_t req = rows[row];
            const int64_t length = lengths[row];
            int32_t found = 0;
            for (int64_t o = 0; o < W; ++o) {
                const int64_t block = topk[(l * B + row) * K + o / bs];
                const int64_t pos = block * bs + o % bs;
                const int valid = block >= 0 && pos < length;
                int in_bounds = valid && req >= 0 && req < R && pos < T;
                int64_t value = -1;
                if (in_bounds) {
                    value = table[((table_layered ? l * R : 0) + req) * T + pos];
                    if (mapping != NULL) {
                        if (value >= 0 && value < N) {
                            value = mapping[(map_layered ? l * N : 0) + value];
                        } else {
                            value = -1;
                            in_bounds = 0;
                        }
                    }
                }
                const int32_t slot = (int32_t)(uint32_t)(uint64_t)value;
                output[(l * B + row) * W + o] = slot;
                if (misses != NULL && in_bounds && slot == 0) {
                    misses[(l * B + row) * W + found] = (int32_t)o;
                    ++found;
                }
            }
            if (counts != NULL) {
                counts[l * B + row] = found;
            }
        }
    }
}

/*
 * Row gather over a fixed-position layout. Follows
 * experimental/sparse_read.py:18-30: valid = 0 <= pos < lengths[b];
 * direct offset = sink + req * request_stride + pos * width;
 * indirect offset = slot_offsets[request_table[req, pos]] (element offsets);
 * invalid rows (and rows that would leave `raw`) are zero.
 */
void oracle_gather_rows(const uint8_t* raw, int64_t raw_elems, int64_t itemsize, const int64_t* positions,
                        int64_t B, int64_t S, const int64_t* request_ids, const int64_t* lengths,
                        const int64_t* request_table, int64_t table_rows, int64_t table_cols,
                        const int64_t* slot_offsets, int64_t slot_len, int indirect, int64_t width,
                        int64_t request_stride, int64_t sink, uint8_t* out) {
    const int64_t row_bytes = width * itemsize;
    for (int64_t b = 0; b < B; ++b) {
        const int64_t req = request_ids[b];
        for (int64_t s = 0; s < S; ++s) {
            const int64_t pos = positions[b * S + s];
            uint8_t* dst = out + (b * S + s) * row_bytes;
            int64_t element = -1;
            if (pos >= 0 && pos < lengths[b]) {
                if (!indirect) {
                    element = sink + req * request_stride + pos * width;
                } else if (req >= 0 && req < table_rows && pos < table_cols) {
                    const int64_t logical = request_table[req * table_cols + pos];
                    if (logical >= 0 && logical < slot_len) {
                        element = slot_offsets[logical];
                    }
                }
            }
            if (element >= 0 && element + width <= raw_elems) {
                memcpy(dst, raw + element * itemsize, (size_t)row_bytes);
            } else {
                memset(dst, 0, (size_t)row_bytes);
            }
        }
    }
}

/*
 * Multi-plane Top-K KV gather (no reference kernel; the indirect gather of
 * experimental/sparse_read.py:11-30 applied per plane):
 *   out[b, l, kv, k, :] = plane(l, kv)[slot] if zero_below <= slot < rows
 *                         else zeros,   slot = slots[l * slot_layer_stride + b * K + k]
 * out is dense [B, L, KV, K, row_bytes]; plane(l, kv) starts at
 * pool + l * layer_stride + kv * kv_stride, slot s at + s * row_stride.
 */
void oracle_gather_kv(const uint8_t* pool, int64_t layer_stride, int64_t kv_stride, int64_t row_stride,
                      int64_t row_bytes, int64_t rows, int64_t L, int64_t B, int64_t KV, int64_t K,
                      const int64_t* slots, int64_t slot_layer_stride, int64_t zero_below, uint8_t* out) {
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t l = 0; l < L; ++l) {
            for (int64_t kv = 0; kv < KV; ++kv) {
                for (int64_t k = 0; k < K; ++k) {
                    const int64_t slot = slots[l * slot_layer_stride + b * K + k];
                    uint8_t* dst = out + (((b * L + l) * KV + kv) * K + k) * row_bytes;
                    if (slot >= zero_below && slot < rows) {
                        memcpy(dst, pool + l * layer_stride + kv * kv_stride + slot * row_stride, (size_t)row_bytes);
                    } else {
                        memset(dst, 0, (size_t)row_bytes);
                    }
                }
            }
        }
    }
}

/* Inverse of oracle_gather_kv: writes only lanes with a valid slot, in lane
 * order (a later lane naming the same slot wins here; the GPU forbids that). */
void oracle_scatter_kv(uint8_t* pool, int64_t layer_stride, int64_t kv_stride, int64_t row_stride,
                       int64_t row_bytes, int64_t rows, int64_t L, int64_t B, int64_t KV, int64_t K,
                       const int64_t* slots, int64_t slot_layer_stride, int64_t zero_below, const uint8_t* src) {
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t l = 0; l < L; ++l) {
            for (int64_t kv = 0; kv < KV; ++kv) {
                for (int64_t k = 0; k < K; ++k) {
                    const int64_t slot = slots[l * slot_layer_stride + b * K + k];
                    if (slot >= zero_below && slot < rows) {
                        memcpy(pool + l * layer_stride + kv * kv_stride + slot * row_stride,
                               src + (((b * L + l) * KV + kv) * K + k) * row_bytes, (size_t)row_bytes);
                    }
                }
            }
        }
    }
}
