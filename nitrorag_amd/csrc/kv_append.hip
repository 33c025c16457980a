// Paged KV append for gfx950: writes new K/V rows into their page slots.
//
// Decode (src/model_q8.cpp:616-623, single sequence :279-287): row b goes to
// page tables[b][pos_b/16], slot pos_b%16, at the layer's offset.
// Prefill scatter (src/model_q8.cpp:473-484): packed row r goes to the slot
// resolved on the host into slots[r] = page*16 + pos%16.
// One float4 per thread (kv_dim is a multiple of 4); page ids outside the pool
// are counted in *bad_pages and skipped.
//
// RoPE + append (src/model_q8.cpp:601-623 decode, :451-484 prefill, :262-287
// single sequence): one workgroup per row rotates each pair (j, j+1) of q (all
// heads) and of k (kv heads) in place by the table entry at
// pos*(head_dim/2) + (j % head_dim)/2 — q' = (q0*c - q1*s, q0*s + q1*c) — and
// writes the rotated k and the unrotated v into the row's page slot.
#include <hip/hip_runtime.h>

#include "device_pool.hpp"

namespace nitro {
namespace {

constexpr int APPEND_THREADS = 256;

// Both append kernels walk the flat (row, float4) index space with a
// grid-stride loop, so any row count runs (rows are not on gridDim.y, whose
// 65,535 limit a large prefill batch would exceed).
__global__ __launch_bounds__(APPEND_THREADS) void kv_append_decode_kernel(
    float* __restrict__ k_pool, float* __restrict__ v_pool, const float* __restrict__ k,
    const float* __restrict__ v, const int32_t* __restrict__ tables,
    const int32_t* __restrict__ positions, int batch, int max_pages, int kv_dim, int64_t page_stride,
    int64_t layer_off, int num_pages, int32_t* bad_pages) {
    const int f4 = kv_dim >> 2;
    const size_t total = (size_t)batch * f4;
    for (size_t t = (size_t)blockIdx.x * APPEND_THREADS + threadIdx.x; t < total;
         t += (size_t)gridDim.x * APPEND_THREADS) {
        const int b = (int)(t / f4), i = (int)(t - (size_t)b * f4);
        const int pos = positions[b];
        const int page = tables[(size_t)b * max_pages + (pos >> 4)];
        if ((unsigned)page >= (unsigned)num_pages) {
            if (i == 0) atomicAdd(bad_pages, 1);
            continue;
        }
        const size_t dst = (size_t)page * page_stride + layer_off + (size_t)(pos & 15) * kv_dim;
        const size_t src = (size_t)b * kv_dim;
        reinterpret_cast<float4*>(k_pool + dst)[i] = reinterpret_cast<const float4*>(k + src)[i];
        reinterpret_cast<float4*>(v_pool + dst)[i] = reinterpret_cast<const float4*>(v + src)[i];
    }
}

__global__ __launch_bounds__(APPEND_THREADS) void kv_scatter_rows_kernel(
    float* __restrict__ k_pool, float* __restrict__ v_pool, const float* __restrict__ k,
    const float* __restrict__ v, const int32_t* __restrict__ slots, int rows, int kv_dim,
    int64_t page_stride, int64_t layer_off, int num_pages, int32_t* bad_pages) {
    const int f4 = kv_dim >> 2;
    const size_t total = (size_t)rows * f4;
    for (size_t t = (size_t)blockIdx.x * APPEND_THREADS + threadIdx.x; t < total;
         t += (size_t)gridDim.x * APPEND_THREADS) {
        const int r = (int)(t / f4), i = (int)(t - (size_t)r * f4);
        const int slot = slots[r];
        const int page = slot >> 4;
        if (slot < 0 || page >= num_pages) {
            if (i == 0) atomicAdd(bad_pages, 1);
            continue;
        }
        const size_t dst = (size_t)page * page_stride + layer_off + (size_t)(slot & 15) * kv_dim;
        const size_t src = (size_t)r * kv_dim;
        reinterpret_cast<float4*>(k_pool + dst)[i] = reinterpret_cast<const float4*>(k + src)[i];
        reinterpret_cast<float4*>(v_pool + dst)[i] = reinterpret_cast<const float4*>(v + src)[i];
    }
}

// Decode rows: position positions[row], page tables[row][pos/16].  Prefill
// rows: position row_pos[row], slot slots[row] (page*16 + pos%16).
__global__ __launch_bounds__(APPEND_THREADS) void rope_kv_append_kernel(
    float* __restrict__ k_pool, float* __restrict__ v_pool, float* __restrict__ q,
    float* __restrict__ k, const float* __restrict__ v, const float* __restrict__ freq_real,
    const float* __restrict__ freq_imag, const int32_t* __restrict__ tables,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ slots,
    const int32_t* __restrict__ row_pos, int max_pages, int dim, int kv_dim, int head_dim,
    int64_t page_stride, int64_t layer_off, int num_pages, int32_t* bad_pages) {
    const int row = blockIdx.x;
    int pos, page, slot_row;
    if (slots) {
        pos = row_pos[row];
        const int slot = slots[row];
        page = slot >> 4;
        slot_row = slot & 15;
    } else {
        pos = positions[row];
        page = tables[(size_t)row * max_pages + (pos >> 4)];
        slot_row = pos & 15;
    }
    const bool page_ok = page >= 0 && page < num_pages;
    if (!page_ok && threadIdx.x == 0) atomicAdd(bad_pages, 1);
    const float* fr = freq_real + (size_t)pos * (head_dim / 2);
    const float* fi = freq_imag + (size_t)pos * (head_dim / 2);
    float2* qrow = reinterpret_cast<float2*>(q + (size_t)row * dim);
    float2* krow = reinterpret_cast<float2*>(k + (size_t)row * kv_dim);
    const float2* vrow = reinterpret_cast<const float2*>(v + (size_t)row * kv_dim);
    float2* kdst = reinterpret_cast<float2*>(k_pool + (size_t)page * page_stride + layer_off +
                                            (size_t)slot_row * kv_dim);
    float2* vdst = reinterpret_cast<float2*>(v_pool + (size_t)page * page_stride + layer_off +
                                            (size_t)slot_row * kv_dim);
    for (int p = threadIdx.x; p < dim / 2; p += APPEND_THREADS) {
        const int f = (2 * p % head_dim) / 2;
        const float c = fr[f], sn = fi[f];
        const float2 x = qrow[p];
        qrow[p] = make_float2(x.x * c - x.y * sn, x.x * sn + x.y * c);
        if (2 * p < kv_dim) {
            const float2 y = krow[p];
            const float2 r = make_float2(y.x * c - y.y * sn, y.x * sn + y.y * c);
            krow[p] = r;
            if (page_ok) {
                kdst[p] = r;
                vdst[p] = vrow[p];
            }
        }
    }
}

}  // namespace

hipError_t launch_rope_kv_append(float* k_pool, float* v_pool, float* q, float* k, const float* v,
                                 const float* freq_real, const float* freq_imag,
                                 const int32_t* tables, const int32_t* positions,
                                 const int32_t* slots, const int32_t* row_pos, int rows,
                                 int max_pages, int dim, int kv_dim, int head_dim,
                                 int64_t page_stride, int64_t layer_off, int num_pages,
                                 int32_t* bad_pages, hipStream_t stream) {
    hipLaunchKernelGGL(rope_kv_append_kernel, dim3(rows), dim3(APPEND_THREADS), 0, stream, k_pool,
                       v_pool, q, k, v, freq_real, freq_imag, tables, positions, slots, row_pos,
                       max_pages, dim, kv_dim, head_dim, page_stride, layer_off, num_pages,
                       bad_pages);
    return hipGetLastError();
}

// Workgroups of the append launches: enough to cover the rows (one float4
// per thread), at most 65,536 (each thread then takes several).
static unsigned append_groups(size_t float4s) {
    const size_t g = (float4s + APPEND_THREADS - 1) / APPEND_THREADS;
    return (unsigned)(g < 1 ? 1 : g > 65536 ? 65536 : g);
}

hipError_t launch_kv_append_decode(float* k_pool, float* v_pool, const float* k, const float* v,
                                   const int32_t* tables, const int32_t* positions, int batch,
                                   int max_pages, int kv_dim, int64_t page_stride,
                                   int64_t layer_off, int num_pages, int32_t* bad_pages,
                                   hipStream_t stream) {
    const dim3 grid(append_groups((size_t)batch * (kv_dim / 4)));
    hipLaunchKernelGGL(kv_append_decode_kernel, grid, dim3(APPEND_THREADS), 0, stream, k_pool,
                       v_pool, k, v, tables, positions, batch, max_pages, kv_dim, page_stride,
                       layer_off, num_pages, bad_pages);
    return hipGetLastError();
}

hipError_t launch_kv_scatter_rows(float* k_pool, float* v_pool, const float* k, const float* v,
                                  const int32_t* slots, int rows, int kv_dim, int64_t page_stride,
                                  int64_t layer_off, int num_pages, int32_t* bad_pages,
                                  hipStream_t stream) {
    const dim3 grid(append_groups((size_t)rows * (kv_dim / 4)));
    hipLaunchKernelGGL(kv_scatter_rows_kernel, grid, dim3(APPEND_THREADS), 0, stream, k_pool,
                       v_pool, k, v, slots, rows, kv_dim, page_stride, layer_off, num_pages,
                       bad_pages);
    return hipGetLastError();
}

}  // namespace nitro
