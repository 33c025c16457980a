// Paged KV append for gfx950: writes new K/V rows into their page slots.
//
// Decode (src/model_q8.cpp:616-623, single sequence :279-287): row b goes to
// page tables[b][pos_b/16], slot pos_b%16, at the layer's offset.
// Prefill scatter (src/model_q8.cpp:473-484): packed row r goes to the slot
// resolved on the host into slots[r] = page*16 + pos%16.
// One float4 per thread (kv_dim is a multiple of 4); page ids outside the pool
// are counted in *bad_pages and skipped.
#include <hip/hip_runtime.h>

#include "device_pool.hpp"

namespace nitro {
namespace {

constexpr int APPEND_THREADS = 256;

__global__ __launch_bounds__(APPEND_THREADS) void kv_append_decode_kernel(
    float* __restrict__ k_pool, float* __restrict__ v_pool, const float* __restrict__ k,
    const float* __restrict__ v, const int32_t* __restrict__ tables,
    const int32_t* __restrict__ positions, int max_pages, int kv_dim, int64_t page_stride,
    int64_t layer_off, int num_pages, int32_t* bad_pages) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * APPEND_THREADS + threadIdx.x;  // float4 index within the row
    if (i * 4 >= kv_dim) return;
    const int pos = positions[b];
    const int page = tables[(size_t)b * max_pages + (pos >> 4)];
    if ((unsigned)page >= (unsigned)num_pages) {
        if (i == 0) atomicAdd(bad_pages, 1);
        return;
    }
    const size_t dst = (size_t)page * page_stride + layer_off + (size_t)(pos & 15) * kv_dim;
    const size_t src = (size_t)b * kv_dim;
    reinterpret_cast<float4*>(k_pool + dst)[i] = reinterpret_cast<const float4*>(k + src)[i];
    reinterpret_cast<float4*>(v_pool + dst)[i] = reinterpret_cast<const float4*>(v + src)[i];
}

__global__ __launch_bounds__(APPEND_THREADS) void kv_scatter_rows_kernel(
    float* __restrict__ k_pool, float* __restrict__ v_pool, const float* __restrict__ k,
    const float* __restrict__ v, const int32_t* __restrict__ slots, int kv_dim,
    int64_t page_stride, int64_t layer_off, int num_pages, int32_t* bad_pages) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * APPEND_THREADS + threadIdx.x;
    if (i * 4 >= kv_dim) return;
    const int slot = slots[r];
    const int page = slot >> 4;
    if (slot < 0 || page >= num_pages) {
        if (i == 0) atomicAdd(bad_pages, 1);
        return;
    }
    const size_t dst = (size_t)page * page_stride + layer_off + (size_t)(slot & 15) * kv_dim;
    const size_t src = (size_t)r * kv_dim;
    reinterpret_cast<float4*>(k_pool + dst)[i] = reinterpret_cast<const float4*>(k + src)[i];
    reinterpret_cast<float4*>(v_pool + dst)[i] = reinterpret_cast<const float4*>(v + src)[i];
}

}  // namespace

hipError_t launch_kv_append_decode(float* k_pool, float* v_pool, const float* k, const float* v,
                                   const int32_t* tables, const int32_t* positions, int batch,
                                   int max_pages, int kv_dim, int64_t page_stride,
                                   int64_t layer_off, int num_pages, int32_t* bad_pages,
                                   hipStream_t stream) {
    const int f4 = kv_dim / 4;
    const dim3 grid((f4 + APPEND_THREADS - 1) / APPEND_THREADS, batch);
    hipLaunchKernelGGL(kv_append_decode_kernel, grid, dim3(APPEND_THREADS), 0, stream, k_pool,
                       v_pool, k, v, tables, positions, max_pages, kv_dim, page_stride, layer_off,
                       num_pages, bad_pages);
    return hipGetLastError();
}

hipError_t launch_kv_scatter_rows(float* k_pool, float* v_pool, const float* k, const float* v,
                                  const int32_t* slots, int rows, int kv_dim, int64_t page_stride,
                                  int64_t layer_off, int num_pages, int32_t* bad_pages,
                                  hipStream_t stream) {
    const int f4 = kv_dim / 4;
    const dim3 grid((f4 + APPEND_THREADS - 1) / APPEND_THREADS, rows);
    hipLaunchKernelGGL(kv_scatter_rows_kernel, grid, dim3(APPEND_THREADS), 0, stream, k_pool,
                       v_pool, k, v, slots, kv_dim, page_stride, layer_off, num_pages, bad_pages);
    return hipGetLastError();
}

}  // namespace nitro
