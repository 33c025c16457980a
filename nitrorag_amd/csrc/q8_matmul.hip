// Q8_0 matrix product for gfx950 (MI355X): out[b][i] = sum_k w[i][k] * x[b][k]
// with w stored as the reference's BlockQ8 rows (src/model_q8.cpp:28-32): per
// 32 consecutive k of a row, a float scale followed by 32 int8 values (36
// bytes), rows of n/32 blocks.  A weight is dequantised as
// float(q) * scale, rounded to fp32 exactly as the reference does
// (src/model_q8.cpp:106-112), and multiplied into fp32 activations; the
// activations are never quantised.
//
// Two semantics, selected per call:
//  - full rows, as matmul (src/model_q8.cpp:92-125);
//  - last block only, as matmul_bulk (src/model_q8.cpp:382-420), whose block
//    loop stores each block's sum over the previous one, so only the final
//    32 columns of every row reach the output.
//
// Layout on the matrix cores (v_mfma_f32_16x16x4_f32, fp32 in, fp32
// accumulate): a workgroup owns 16 output rows; out^T[16 rows][16 batch] +=
// W[16 rows][4 k] . x^T[4 k][16 batch] per instruction.  Per 64-k chunk (two
// blocks), lane l = (r = l%16, g = l/16) loads the 16 int8 of row r in half
// g%2 of block 2*chunk + g/2 (one 16-byte run) and that block's scale; MFMA
// m (0..15) takes the lane's m-th weight, so the k-slot g of instruction m is
// k = (2*chunk + g/2)*32 + (g%2)*16 + m, and the B operand lane (c, g) holds
// x[c][that k] (16 contiguous floats per lane).  The four waves take chunks
// round-robin and add their partial tiles through LDS.  Batches of more than
// 16 rows reuse the dequantised weights for every 16-row batch tile.
#include <hip/hip_runtime.h>

#include "device_pool.hpp"

namespace nitro {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int Q8_BLOCK = 32;         // weights per block
constexpr int Q8_BLOCK_BYTES = 36;   // float scale + 32 int8
constexpr int Q8_WAVES = 4;
constexpr int Q8_MAX_BTILES = 4;     // batch tiles of 16 per launch row (batch <= 64 per grid.y)

__device__ __forceinline__ float dequant(uint32_t q4, int j, float scale) {
    return (float)(int)(int8_t)(q4 >> (8 * j)) * scale;
}

template <bool LAST_BLOCK_ONLY>
__global__ __launch_bounds__(64 * Q8_WAVES) void q8_matmul_kernel(const uint8_t* __restrict__ w,
                                                                   const float* __restrict__ x,
                                                                   float* __restrict__ out,
                                                                   int batch, int n, int d) {
    __shared__ f32x4 red[Q8_WAVES - 1][Q8_MAX_BTILES][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int row0 = blockIdx.x * 16;
    const int b0 = blockIdx.y * 16 * Q8_MAX_BTILES;  // first batch row of this launch row
    const int btiles = min(Q8_MAX_BTILES, (batch - b0 + 15) / 16);
    const int nb = n / Q8_BLOCK;
    const int nchunk = (nb + 1) / 2;
    const uint8_t* wrow = w + (size_t)min(row0 + r, d - 1) * nb * Q8_BLOCK_BYTES;

    f32x4 acc[Q8_MAX_BTILES];
#pragma unroll
    for (int t = 0; t < Q8_MAX_BTILES; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int first = LAST_BLOCK_ONLY ? nchunk - 1 : 0;
    for (int ch = first + wave; ch < nchunk; ch += Q8_WAVES) {
        const int blk = 2 * ch + (g >> 1);
        const int half = g & 1;
        const bool valid = blk < nb && (!LAST_BLOCK_ONLY || blk == nb - 1);
        float wv[16];
        if (valid) {
            const uint8_t* bp = wrow + (size_t)blk * Q8_BLOCK_BYTES;
            const float scale = *reinterpret_cast<const float*>(bp);
            const uint32_t* qp = reinterpret_cast<const uint32_t*>(bp + 4 + 16 * half);
            const uint32_t q0 = qp[0], q1 = qp[1], q2 = qp[2], q3 = qp[3];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                wv[j] = dequant(q0, j, scale);
                wv[4 + j] = dequant(q1, j, scale);
                wv[8 + j] = dequant(q2, j, scale);
                wv[12 + j] = dequant(q3, j, scale);
            }
        } else {
#pragma unroll
            for (int m = 0; m < 16; m++) wv[m] = 0.0f;
        }
        const int k0 = blk * Q8_BLOCK + 16 * half;
#pragma unroll
        for (int t = 0; t < Q8_MAX_BTILES; t++) {
            if (t < btiles) {  // uniform
                const int bb = b0 + t * 16 + r;  // batch row this lane feeds (B operand column)
                float xv[16];
                if (valid && bb < batch) {
                    const float4* xp = reinterpret_cast<const float4*>(x + (size_t)bb * n + k0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float4 v = xp[i];
                        xv[4 * i] = v.x;
                        xv[4 * i + 1] = v.y;
                        xv[4 * i + 2] = v.z;
                        xv[4 * i + 3] = v.w;
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < 16; m++) xv[m] = 0.0f;
                }
#pragma unroll
                for (int m = 0; m < 16; m++)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[m], xv[m], acc[t], 0, 0, 0);
            }
        }
    }

    // Sum the four waves' partial tiles; wave 0 writes.  Lane l holds
    // out^T[row0 + 4*(l/16) + j][b0 + 16t + l%16], j = 0..3.
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < Q8_MAX_BTILES; t++)
            if (t < btiles) red[wave - 1][t][lane] = acc[t];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int t = 0; t < Q8_MAX_BTILES; t++) {
        if (t >= btiles) break;
        f32x4 s = acc[t];
#pragma unroll
        for (int v = 0; v < Q8_WAVES - 1; v++) s += red[v][t][lane];
        const int bb = b0 + t * 16 + (lane & 15);
        if (bb >= batch) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = row0 + 4 * (lane >> 4) + j;
            if (row < d) out[(size_t)bb * d + row] = s[j];
        }
    }
}

}  // namespace

hipError_t launch_q8_matmul(const void* w, const float* x, float* out, int batch, int n, int d,
                            bool last_block_only, hipStream_t stream) {
    const dim3 grid((unsigned)((d + 15) / 16), (unsigned)((batch + 16 * Q8_MAX_BTILES - 1) / (16 * Q8_MAX_BTILES)));
    const dim3 block(64 * Q8_WAVES);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (last_block_only)
        hipLaunchKernelGGL(q8_matmul_kernel<true>, grid, block, 0, stream, wb, x, out, batch, n, d);
    else
        hipLaunchKernelGGL(q8_matmul_kernel<false>, grid, block, 0, stream, wb, x, out, batch, n, d);
    return hipGetLastError();
}

}  // namespace nitro
