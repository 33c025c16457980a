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
//
// Batches of 1..4 rows use a VALU form of the same lane layout (q8_gemv):
// each lane forms the dot products of its 16 weights with x directly, the
// four lane groups of a row are summed with gfx950's row-swap permutes and
// the waves through LDS.  Both kernels issue the weight loads of Q8_UNROLL
// chunks before using any, so enough HBM reads are in flight per wave.
#include <hip/hip_runtime.h>

#include "device_pool.hpp"

namespace nitro {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int Q8_BLOCK = 32;         // weights per block
constexpr int Q8_BLOCK_BYTES = 36;   // float scale + 32 int8
constexpr int Q8_WAVES = 4;
constexpr int Q8_MAX_BTILES = 4;     // batch tiles of 16 per launch row (batch <= 64 per grid.y)
constexpr int Q8_UNROLL = 4;         // 64-weight chunks whose loads a wave issues together
constexpr int Q8_GEMV_MAX_BATCH = 4;

// The 16 int8 weights and the scale a lane feeds for one 64-k chunk.
struct Q8Slice {
    uint32_t q[4];
    float scale;
};

__device__ __forceinline__ Q8Slice load_slice(const uint8_t* wrow, int blk, int half, bool valid) {
    Q8Slice s{{0u, 0u, 0u, 0u}, 0.0f};
    if (valid) {
        const uint8_t* bp = wrow + (size_t)blk * 36;
        s.scale = *reinterpret_cast<const float*>(bp);
        const uint32_t* qp = reinterpret_cast<const uint32_t*>(bp + 4 + 16 * half);
        s.q[0] = qp[0];
        s.q[1] = qp[1];
        s.q[2] = qp[2];
        s.q[3] = qp[3];
    }
    return s;
}

__device__ __forceinline__ float sum_over_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

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
    // Wave w takes chunks first + (round*Q8_WAVES + w)*Q8_UNROLL + u.
    for (int base = first + wave * Q8_UNROLL; base < nchunk; base += Q8_WAVES * Q8_UNROLL) {
        Q8Slice sl[Q8_UNROLL];
#pragma unroll
        for (int u = 0; u < Q8_UNROLL; u++) {
            const int blk = 2 * (base + u) + (g >> 1);
            const bool valid = base + u < nchunk && blk < nb && (!LAST_BLOCK_ONLY || blk == nb - 1);
            sl[u] = load_slice(wrow, blk, g & 1, valid);
        }
#pragma unroll
        for (int u = 0; u < Q8_UNROLL; u++) {
            if (base + u >= nchunk) break;  // uniform
            const int blk = 2 * (base + u) + (g >> 1);
            const bool valid = blk < nb && (!LAST_BLOCK_ONLY || blk == nb - 1);
            float wv[16];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                wv[j] = dequant(sl[u].q[0], j, sl[u].scale);
                wv[4 + j] = dequant(sl[u].q[1], j, sl[u].scale);
                wv[8 + j] = dequant(sl[u].q[2], j, sl[u].scale);
                wv[12 + j] = dequant(sl[u].q[3], j, sl[u].scale);
            }
            const int k0 = blk * Q8_BLOCK + 16 * (g & 1);
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

// Batches of 1..NB rows on the VALU: lane (r, g) dots its 16 weights of row
// row0 + r with x[b] at the same 16 k for every b.  A workgroup of
// GEMV_WAVES waves owns 16 rows; per slab of GEMV_WAVES*Q8_UNROLL chunks
// (2048 k) each wave first issues the weight loads of its Q8_UNROLL chunks,
// then the workgroup stages the slab of x in LDS (lanes of a lane group read
// the same x, which LDS broadcasts), and then the waves compute.  The 4 lane
// groups are summed with row-swap permutes and the waves through LDS in a
// fixed order (results are repeatable bit for bit).
constexpr int GEMV_WAVES = 8;
constexpr int GEMV_SLAB = GEMV_WAVES * Q8_UNROLL * 64;  // k per slab

template <int NB, bool LAST_BLOCK_ONLY>
__global__ __launch_bounds__(64 * GEMV_WAVES) void q8_gemv_kernel(const uint8_t* __restrict__ w,
                                                                   const float* __restrict__ x,
                                                                   float* __restrict__ out, int n, int d) {
    __shared__ __attribute__((aligned(16))) float xs[NB][GEMV_SLAB];
    __shared__ float red[GEMV_WAVES][NB][16];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int row0 = blockIdx.x * 16;
    const int nb = n / Q8_BLOCK;
    const int nchunk = (nb + 1) / 2;
    const uint8_t* wrow = w + (size_t)min(row0 + r, d - 1) * nb * Q8_BLOCK_BYTES;

    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = 0.0f;

    // In the last-block form only the final chunk matters: one slab holding it.
    const int k_begin = LAST_BLOCK_ONLY ? (nchunk - 1) * 64 : 0;
    for (int slab = k_begin; slab < n; slab += GEMV_SLAB) {
        const int c0 = slab / 64 + wave * Q8_UNROLL;  // this wave's first chunk
        Q8Slice sl[Q8_UNROLL];
#pragma unroll
        for (int u = 0; u < Q8_UNROLL; u++) {
            const int blk = 2 * (c0 + u) + (g >> 1);
            const bool valid = c0 + u < nchunk && blk < nb && (!LAST_BLOCK_ONLY || blk == nb - 1);
            sl[u] = load_slice(wrow, blk, g & 1, valid);
        }
        const int slab_len = min(GEMV_SLAB, n - slab);  // multiple of 32
        __syncthreads();  // previous slab's x reads are done
        for (int i = threadIdx.x; i < NB * (slab_len / 4); i += 64 * GEMV_WAVES) {
            const int b = i / (slab_len / 4), f = i - b * (slab_len / 4);
            *reinterpret_cast<float4*>(&xs[b][4 * f]) =
                reinterpret_cast<const float4*>(x + (size_t)b * n + slab)[f];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < Q8_UNROLL; u++) {
            const int blk = 2 * (c0 + u) + (g >> 1);
            const bool valid = c0 + u < nchunk && blk < nb && (!LAST_BLOCK_ONLY || blk == nb - 1);
            if (!valid) continue;  // no cross-lane work inside the chunk loop
            const int kl = blk * Q8_BLOCK + 16 * (g & 1) - slab;  // k within the slab
            float wv[16];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                wv[j] = dequant(sl[u].q[0], j, sl[u].scale);
                wv[4 + j] = dequant(sl[u].q[1], j, sl[u].scale);
                wv[8 + j] = dequant(sl[u].q[2], j, sl[u].scale);
                wv[12 + j] = dequant(sl[u].q[3], j, sl[u].scale);
            }
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const float4* xp = reinterpret_cast<const float4*>(&xs[b][kl]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 v = xp[i];
                    acc[b] = fmaf(wv[4 * i], v.x, acc[b]);
                    acc[b] = fmaf(wv[4 * i + 1], v.y, acc[b]);
                    acc[b] = fmaf(wv[4 * i + 2], v.z, acc[b]);
                    acc[b] = fmaf(wv[4 * i + 3], v.w, acc[b]);
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = sum_over_rows(acc[b]);  // lanes r, r+16, r+32, r+48
    if (g == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) red[wave][b][r] = acc[b];
    }
    __syncthreads();
    if (threadIdx.x >= NB * 16) return;
    const int b = threadIdx.x / 16, rr = threadIdx.x % 16;
    if (row0 + rr >= d) return;
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < GEMV_WAVES; v++) sum += red[v][b][rr];
    out[(size_t)b * d + row0 + rr] = sum;
}

template <int NB>
static void launch_gemv(const uint8_t* w, const float* x, float* out, int n, int d, bool last,
                        hipStream_t stream) {
    const dim3 grid((unsigned)((d + 15) / 16)), block(64 * GEMV_WAVES);
    if (last)
        hipLaunchKernelGGL((q8_gemv_kernel<NB, true>), grid, block, 0, stream, w, x, out, n, d);
    else
        hipLaunchKernelGGL((q8_gemv_kernel<NB, false>), grid, block, 0, stream, w, x, out, n, d);
}

}  // namespace

hipError_t launch_q8_matmul(const void* w, const float* x, float* out, int batch, int n, int d,
                            bool last_block_only, hipStream_t stream) {
    const dim3 grid((unsigned)((d + 15) / 16), (unsigned)((batch + 16 * Q8_MAX_BTILES - 1) / (16 * Q8_MAX_BTILES)));
    const dim3 block(64 * Q8_WAVES);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (batch <= Q8_GEMV_MAX_BATCH) {
        switch (batch) {
            case 1: launch_gemv<1>(wb, x, out, n, d, last_block_only, stream); break;
            case 2: launch_gemv<2>(wb, x, out, n, d, last_block_only, stream); break;
            case 3: launch_gemv<3>(wb, x, out, n, d, last_block_only, stream); break;
            default: launch_gemv<4>(wb, x, out, n, d, last_block_only, stream); break;
        }
        return hipGetLastError();
    }
    if (last_block_only)
        hipLaunchKernelGGL(q8_matmul_kernel<true>, grid, block, 0, stream, wb, x, out, batch, n, d);
    else
        hipLaunchKernelGGL(q8_matmul_kernel<false>, grid, block, 0, stream, wb, x, out, batch, n, d);
    return hipGetLastError();
}

}  // namespace nitro
