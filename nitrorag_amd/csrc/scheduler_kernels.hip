// Device kernels of the continuous scheduler's step for gfx950.
//  - sched_tables: keeps one block-table row per request resident on the
//    device and writes this step's decode tables from it.  Each decode row
//    brings at most one new page (one token per step); pages that other
//    requests gained this step (prefix hits, prefill chunks) arrive as a list
//    of (row * row_stride + index, page) pairs.  Rows of a short prefill
//    chunk taken into the decode batch read the chunk's uploaded table.
//    Nothing but the new entries (and such a chunk's table) crosses PCIe.
//  - argmax_rows: the reference's argmax (src/model_q8.cpp:559-569) per row:
//    the first index of the largest value above 0.0, index 0 when no value
//    exceeds 0.0 (NaN never wins).
#include <hip/hip_runtime.h>

#include "device_pool.hpp"

namespace nitro {
namespace {

constexpr int SCHED_THREADS = 256;

// Workgroup b < batch: row b of the decode batch, desc[b] = {slot, position,
// new index or -1, new page}.  A request's row (slot >= 0) records its new
// page in the resident row; a prefill-chunk row (slot -1) reads the chunk's
// uploaded table instead.  Either writes tables[b][0, max_pages) (entries
// past the position's page are 0), positions[b] and slots[b] = page * 16 +
// position % 16 (where the row's K/V goes).  Workgroup `batch`
// (present when n_other > 0) stores the new entries of requests that are
// not decode rows; no row of this launch reads those.
__global__ __launch_bounds__(SCHED_THREADS) void sched_tables_kernel(
    int32_t* __restrict__ store, int row_stride, const int32_t* __restrict__ desc,
    const int32_t* __restrict__ other, int n_other, const int32_t* __restrict__ chunk_table,
    int32_t* __restrict__ tables, int32_t* __restrict__ positions, int32_t* __restrict__ slots, int batch,
    int max_pages) {
    const int b = blockIdx.x;
    if (b == batch) {
        for (int i = threadIdx.x; i < n_other; i += SCHED_THREADS) store[other[2 * i]] = other[2 * i + 1];
        return;
    }
    const int slot = desc[4 * b], pos = desc[4 * b + 1], new_idx = desc[4 * b + 2], new_page = desc[4 * b + 3];
    const int32_t* row = slot >= 0 ? store + (size_t)slot * row_stride : chunk_table;
    if (threadIdx.x == 0) {
        if (slot >= 0 && new_idx >= 0) store[(size_t)slot * row_stride + new_idx] = new_page;
        positions[b] = pos;
        const int j = pos >> 4;  // the row's own page: new this step, or already resident
        slots[b] = ((j == new_idx) ? new_page : row[j]) * 16 + (pos & 15);
    }
    const int pages = (pos >> 4) + 1;
    int32_t* out = tables + (size_t)b * max_pages;
    for (int j = threadIdx.x; j < max_pages; j += SCHED_THREADS)
        out[j] = j < pages ? (j == new_idx ? new_page : row[j]) : 0;
}

// (value, index) of the reference's argmax over a subset: strict '>' keeps the
// first index of equal values; the start (0.0, 0) is the reference's.
struct Best {
    float v;
    int i;
};

__device__ __forceinline__ Best better(Best a, Best b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

// One 1024-thread workgroup per row; rows of a multiple of 4 floats are read
// as float4 with every load of a thread issued before its compares (a 32000-
// entry row is ~8 loads per thread).  Each thread scans its elements in
// increasing index order, so its candidate is the first index of its maximum.
constexpr int ARGMAX_THREADS = 1024;

__global__ __launch_bounds__(ARGMAX_THREADS) void argmax_rows_kernel(const float* __restrict__ logits,
                                                                     int32_t* __restrict__ next, int vocab) {
    __shared__ Best red[ARGMAX_THREADS / 64];
    const float* row = logits + (size_t)blockIdx.x * vocab;
    Best best{0.0f, 0};
    if ((vocab & 3) == 0) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
        const int n4 = vocab >> 2;
        constexpr int U = 8;
        for (int base = threadIdx.x; base < n4; base += U * ARGMAX_THREADS) {
            float4 v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int j = base + u * ARGMAX_THREADS;
                v[u] = j < n4 ? r4[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = 4 * (base + u * ARGMAX_THREADS);
                if (v[u].x > best.v) best = Best{v[u].x, i};
                if (v[u].y > best.v) best = Best{v[u].y, i + 1};
                if (v[u].z > best.v) best = Best{v[u].z, i + 2};
                if (v[u].w > best.v) best = Best{v[u].w, i + 3};
            }
        }
    } else {
        for (int i = threadIdx.x; i < vocab; i += ARGMAX_THREADS) {
            const float v = row[i];
            if (v > best.v) best = Best{v, i};
        }
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        Best o{__shfl_xor(best.v, m), __shfl_xor(best.i, m)};
        best = better(best, o);
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        Best r = red[0];
#pragma unroll
        for (int w = 1; w < ARGMAX_THREADS / 64; w++) r = better(r, red[w]);
        next[blockIdx.x] = r.i;
    }
}

}  // namespace

hipError_t launch_sched_tables(int32_t* store, int row_stride, const int32_t* desc, const int32_t* other,
                               int n_other, const int32_t* chunk_table, int32_t* tables, int32_t* positions,
                               int32_t* slots, int batch, int max_pages, hipStream_t stream) {
    const int groups = batch + (n_other > 0 ? 1 : 0);
    if (groups == 0) return hipSuccess;
    hipLaunchKernelGGL(sched_tables_kernel, dim3(groups), dim3(SCHED_THREADS), 0, stream, store, row_stride,
                       desc, other, n_other, chunk_table, tables, positions, slots, batch, max_pages);
    return hipGetLastError();
}

hipError_t launch_argmax_rows(const float* logits, int32_t* next, int rows, int vocab, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(ARGMAX_THREADS), 0, stream, logits, next, vocab);
    return hipGetLastError();
}

}  // namespace nitro
