// Row-wise kernels of the transformer step around attention for gfx950, and
// the fp32 matrix product of the classifier.  Each follows the reference's
// formula (src/model_q8.cpp); reductions run in parallel, so sums differ from
// the reference's sequential order by fp32 rounding only.
//  - embed_rows: x[r] = token_embedding_table[tokens[r]] (:573-580, :432-436)
//  - add_rmsnorm: x[r] += delta[r] (optional), then
//      out[r] = weight * (x[r] / sqrtf(mean(x[r]^2) + 1e-5))  (rms_norm, :128-140)
//  - swiglu: hb = hb * (1 / (1 + expf(-hb))) * hb2  (:672-680, :536-544)
//  - f32_matmul: out[b][i] = sum_k w[i][k] * x[b][k], w fp32 [d][n]
//      (matmul :80-90 and matmul_bulk :370-380, float overloads: the
//      classifier wcls), VALU for up to 4 rows, fp32 MFMA above.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "device_pool.hpp"

namespace nitro {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int ROW_THREADS = 256;

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < ROW_THREADS / 64; w++) s += red[w];
    return s;
}

__global__ __launch_bounds__(ROW_THREADS) void embed_rows_kernel(const float* __restrict__ table,
                                                                 const int32_t* __restrict__ tokens,
                                                                 float* __restrict__ x, int dim,
                                                                 int vocab, int32_t* bad_tokens,
                                                                 float* __restrict__ ss) {
    __shared__ float red[ROW_THREADS / 64];
    const int r = blockIdx.x;
    int t = tokens[r];
    if ((unsigned)t >= (unsigned)vocab) {
        if (threadIdx.x == 0) atomicAdd(bad_tokens, 1);
        t = 0;  // defined result; the count reports the bad id
    }
    const float4* src = reinterpret_cast<const float4*>(table + (size_t)t * dim);
    float4* dst = reinterpret_cast<float4*>(x + (size_t)r * dim);
    float sq = 0.0f;
    for (int i = threadIdx.x; i < dim / 4; i += ROW_THREADS) {
        const float4 v = src[i];
        dst[i] = v;
        sq = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, sq))));
    }
    if (ss) {  // uniform
        sq = block_sum(sq, red);
        if (threadIdx.x == 0) ss[r] = sq;
    }
}

// One workgroup per row; x, delta, out are [rows][dim] (out may alias x).
__global__ __launch_bounds__(ROW_THREADS) void add_rmsnorm_kernel(float* x,
                                                                  const float* __restrict__ delta,
                                                                  const float* __restrict__ weight,
                                                                  float* out, int dim) {
    __shared__ float red[ROW_THREADS / 64];
    float* xr = x + (size_t)blockIdx.x * dim;
    const float* dr = delta ? delta + (size_t)blockIdx.x * dim : nullptr;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < dim; i += ROW_THREADS) {
        float v = xr[i];
        if (dr) {
            v += dr[i];
            xr[i] = v;
        }
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)dim + 1e-5f);
    float* orow = out + (size_t)blockIdx.x * dim;
    for (int i = threadIdx.x; i < dim; i += ROW_THREADS) orow[i] = weight[i] * (inv * xr[i]);
}

// last[b] = x[r] (+ ffn[r] when given) for the last row r = row_off[b] + len[b] - 1 of chunk b.
__global__ __launch_bounds__(ROW_THREADS) void gather_last_rows_kernel(const float* __restrict__ x,
                                                                       const float* __restrict__ ffn,
                                                                       const int32_t* __restrict__ row_off,
                                                                       const int32_t* __restrict__ len,
                                                                       float* __restrict__ last, int dim) {
    const int b = blockIdx.x;
    const size_t r = (size_t)(row_off[b] + len[b] - 1);
    for (int i = threadIdx.x; i < dim; i += ROW_THREADS)
        last[(size_t)b * dim + i] = ffn ? x[r * dim + i] + ffn[r * dim + i] : x[r * dim + i];
}

__global__ __launch_bounds__(ROW_THREADS) void swiglu_kernel(float* __restrict__ hb,
                                                             const float* __restrict__ hb2, size_t n) {
    const size_t i = (size_t)blockIdx.x * ROW_THREADS + threadIdx.x;
    if (i >= n) return;
    float v = hb[i];
    v *= 1.0f / (1.0f + expf(-v));
    hb[i] = v * hb2[i];
}

// fp32 rows of w: lane (r = l%16, g = l/16) takes k = 64*chunk + 16*g .. +15
// of row row0 + r (64 contiguous bytes); same lane layout as the Q8 kernels.
constexpr int F32_WAVES = 8;
constexpr int F32_UNROLL = 2;
constexpr int F32_SLAB = F32_WAVES * F32_UNROLL * 64;

__device__ __forceinline__ float sum_over_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Up to NB activation rows on the VALU; n % 64 == 0.
template <int NB>
__global__ __launch_bounds__(64 * F32_WAVES) void f32_gemv_kernel(const float* __restrict__ w,
                                                                   const float* __restrict__ x,
                                                                   float* __restrict__ out, int n, int d) {
    __shared__ __attribute__((aligned(16))) float xs[NB][F32_SLAB];
    __shared__ float red[F32_WAVES][NB][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int row0 = blockIdx.x * 16;
    const float* wrow = w + (size_t)min(row0 + r, d - 1) * n;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = 0.0f;
    for (int slab = 0; slab < n; slab += F32_SLAB) {
        const int k0 = slab + wave * F32_UNROLL * 64 + 16 * g;
        float4 wv[F32_UNROLL][4];
#pragma unroll
        for (int u = 0; u < F32_UNROLL; u++) {
            const int k = k0 + 64 * u;
#pragma unroll
            for (int i = 0; i < 4; i++)
                wv[u][i] = k < n ? reinterpret_cast<const float4*>(wrow + k)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const int slab_len = min(F32_SLAB, n - slab);
        __syncthreads();
        for (int i = threadIdx.x; i < NB * (slab_len / 4); i += 64 * F32_WAVES) {
            const int b = i / (slab_len / 4), f = i - b * (slab_len / 4);
            *reinterpret_cast<float4*>(&xs[b][4 * f]) = reinterpret_cast<const float4*>(x + (size_t)b * n + slab)[f];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < F32_UNROLL; u++) {
            const int k = k0 + 64 * u;
            if (k >= n) continue;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const float4* xp = reinterpret_cast<const float4*>(&xs[b][k - slab]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 v = xp[i];
                    acc[b] = fmaf(wv[u][i].x, v.x, acc[b]);
                    acc[b] = fmaf(wv[u][i].y, v.y, acc[b]);
                    acc[b] = fmaf(wv[u][i].z, v.z, acc[b]);
                    acc[b] = fmaf(wv[u][i].w, v.w, acc[b]);
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = sum_over_rows(acc[b]);
    if (g == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) red[wave][b][r] = acc[b];
    }
    __syncthreads();
    if (threadIdx.x >= NB * 16) return;
    const int b = threadIdx.x / 16, rr = threadIdx.x % 16;
    if (row0 + rr >= d) return;
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < F32_WAVES; v++) s += red[v][b][rr];
    out[(size_t)b * d + row0 + rr] = s;
}

// Up to NB activation rows whose x fits LDS (NB * n <= F32F_X_MAX floats):
// x is staged in LDS once per workgroup, so a wave's only loads from memory
// in its loop are weights and the next item's stay in flight while the
// current one is used.  Persistent workgroups own balanced ranges of 2-row
// groups; items are (group, 1024-k chunk), split between the 8 waves in
// contiguous runs.  Lane l takes float4 l, l + 64, l + 128, l + 192 of the
// chunk in both rows, so each load instruction reads 1 KB of a row
// contiguously.  At a group's last chunk (or the end of the wave's run) each
// row's 64 lanes are summed with a fixed butterfly into the wave's LDS slot;
// the slots are added in wave order.
// NORM (the final rms_norm folded in, nm as for the Q8 products): x is staged
// times the norm weights and each row sum is scaled by the row's 1/rms,
// summed from the partial sums of squares the last residual product left
// (src/model_q8.cpp:687-692 normalises x first; the two agree to fp32
// rounding).  The prologue's loads go out x first, then the partials, then
// the first item's weights, so the waits for x and the partials leave the
// weights in flight.
// NT: the weights are read with non-temporal loads, for a matrix larger than
// the 256 MB Infinity Cache (nothing of it survives to the next step): the
// Llama-2-7B-shaped classifier (32000 x 4096) took 84.2 us against 90.5 with
// plain loads.  A smaller one (the 110M-shaped classifier, 98 MB) keeps plain
// loads, so what the cache holds between steps can serve it.
constexpr int F32F_WAVES = 8;
constexpr int F32F_X_MAX = 16384;
constexpr size_t F32F_NT_MIN_BYTES = 256ull << 20;

template <int NB, bool NORM, bool NT_W>
__global__ __launch_bounds__(64 * F32F_WAVES) void f32_flat_kernel(const float* __restrict__ w,
                                                                   const float* __restrict__ x,
                                                                   float* __restrict__ out, int n, int d,
                                                                   Q8Norm nm) {
    constexpr int W = F32F_WAVES, NT = 64 * W, R = 2, PE = 4;
    // [NB][n] x, then [rows][NB][W] sums, then [NB] 1/rms
    extern __shared__ __attribute__((aligned(16))) float f32f_lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nch = (n + 1023) / 1024;
    const int groups = (d + R - 1) / R;
    const int g0 = (int)((long long)groups * blockIdx.x / gridDim.x);
    const int g1 = (int)((long long)groups * (blockIdx.x + 1) / gridDim.x);
    const int items = (g1 - g0) * nch;
    const int i0 = items * wave / W, i1 = items * (wave + 1) / W;
    const int rows = (g1 - g0) * R;
    float* xs = f32f_lds;
    float* red = f32f_lds + NB * n;
    float* inv_s = red + rows * NB * W;
    auto load_item = [&](float4 (&v)[R][4], int i) {
        i = max(min(i, i1 - 1), 0);  // clamped into the run: a wave with no items loads in range, never used
        const int g = g0 + i / nch, c = i % nch;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float* rowp = w + (size_t)min(g * R + r, d - 1) * n;
#pragma unroll
            for (int q = 0; q < 4; q++) {  // past the row: the last float4 again (its x are zeroed)
                const float* p = rowp + min(1024 * c + 4 * lane + 256 * q, n - 4);
                if constexpr (NT_W)
                    v[r][q] = __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p)));
                else
                    v[r][q] = *reinterpret_cast<const float4*>(p);
            }
        }
    };
    // x (and the norm weights): NB * n / 4 float4, at most 2 per thread for a
    // 4096-wide row at NB <= 2 (XV per thread in all)
    constexpr int XV = (F32F_X_MAX / 4 + NT - 1) / NT;
    const int total = NB * n / 4;
    float4 xr[XV], wr[XV];
#pragma unroll
    for (int v = 0; v < XV; v++) {
        const int t = min((int)threadIdx.x + v * NT, total - 1);
        if ((int)threadIdx.x + v * NT < total) {
            xr[v] = reinterpret_cast<const float4*>(x)[t];
            if constexpr (NORM) wr[v] = reinterpret_cast<const float4*>(nm.weight)[t % (n / 4)];
        }
    }
    float pv[PE];
    if constexpr (NORM) {
        const int pb = min(wave, NB - 1);
#pragma unroll
        for (int k = 0; k < PE; k++) pv[k] = nm.ss[(size_t)min(lane + k * 64, nm.nparts - 1) * nm.ss_stride + pb];
    }
    float4 va[R][4], vb[R][4];
    __builtin_amdgcn_sched_barrier(0);  // (left free, the scheduler issues the weights first)
    load_item(va, i0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int v = 0; v < XV; v++) {
        const int t = (int)threadIdx.x + v * NT;
        if (t < total) {
            float4 o = xr[v];
            if constexpr (NORM) o = make_float4(wr[v].x * o.x, wr[v].y * o.y, wr[v].z * o.z, wr[v].w * o.w);
            reinterpret_cast<float4*>(xs)[t] = o;
        }
    }
    for (int t = threadIdx.x; t < rows * NB * W; t += NT) red[t] = 0.0f;
    __syncthreads();
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[r][b] = 0.0f;
    auto step = [&](const float4 (&now)[R][4], float4 (&next)[R][4], int i) {
        load_item(next, i + 1);
        const int gl = i / nch, c = i % nch;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float4 xv[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int k = 1024 * c + 4 * lane + 256 * q;
                const float4 t = *reinterpret_cast<const float4*>(xs + b * n + (k < n ? k : 0));
                xv[q] = k < n ? t : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    acc[r][b] = fmaf(now[r][q].x, xv[q].x, acc[r][b]);
                    acc[r][b] = fmaf(now[r][q].y, xv[q].y, acc[r][b]);
                    acc[r][b] = fmaf(now[r][q].z, xv[q].z, acc[r][b]);
                    acc[r][b] = fmaf(now[r][q].w, xv[q].w, acc[r][b]);
                }
        }
        if (c == nch - 1 || i == i1 - 1) {  // wave-uniform
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    float v = acc[r][b];
#pragma unroll
                    for (int msk = 32; msk > 0; msk >>= 1) v += __shfl_xor(v, msk);
                    if (lane == 0) red[((gl * R + r) * NB + b) * W + wave] = v;
                    acc[r][b] = 0.0f;
                }
        }
    };
    int i = i0;
    for (; i + 1 < i1; i += 2) {
        step(va, vb, i);
        step(vb, va, i + 1);
    }
    if (i < i1) step(va, vb, i);
    if constexpr (NORM) {
        // wave b < NB adds batch row b's partials in order (as the Q8 products do)
        if (wave < NB) {
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < PE; k++) v += lane + k * 64 < nm.nparts ? pv[k] : 0.0f;
            for (int p = lane + PE * 64; p < nm.nparts; p += 64) v += nm.ss[(size_t)p * nm.ss_stride + wave];
#pragma unroll
            for (int msk = 32; msk > 0; msk >>= 1) v += __shfl_xor(v, msk);
            if (lane == 0) inv_s[wave] = 1.0f / sqrtf(v / (float)n + 1e-5f);
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < NB * rows; t += NT) {
        const int b = t / rows, il = t - b * rows;
        const int row = g0 * R + il;
        float v = 0.0f;
#pragma unroll
        for (int ww = 0; ww < W; ww++) v += red[(il * NB + b) * W + ww];
        if (row < d) out[(size_t)b * d + row] = NORM ? v * inv_s[b] : v;
    }
}

// More rows on fp32 MFMA: out^T[16 rows][16 batch] per wave and tile pair, 4
// waves split k by 64-k chunks; lane (r, g) feeds w[row][64c + 16g + m] and
// x[b][64c + 16g + m] to instruction m.  A workgroup takes RT 16-row tiles,
// so each x value a lane loads serves that many rows' products: two for two
// or more batch tiles (with one, the x reads from L2 were twice the weight
// reads from HBM: the Llama-2-110M classifier, 32000 x 768 at batch 32, 37.7
// against 31.7 us), one otherwise (the 7B classifier, 32000 x 4096 at batch
// 8, took 129 us with two, 113 with one: half the workgroups).
constexpr int F32M_WAVES = 4;
constexpr int F32M_BTILES = 4;

template <int F32M_RTILES>
__global__ __launch_bounds__(64 * F32M_WAVES) void f32_matmul_mfma_kernel(const float* __restrict__ w,
                                                                          const float* __restrict__ x,
                                                                          float* __restrict__ out,
                                                                          int batch, int n, int d) {
    __shared__ f32x4 red[F32M_WAVES - 1][F32M_RTILES][F32M_BTILES][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int row0 = blockIdx.x * 16 * F32M_RTILES;
    const int b0 = blockIdx.y * 16 * F32M_BTILES;
    const int btiles = min(F32M_BTILES, (batch - b0 + 15) / 16);
    const float* wrow[F32M_RTILES];
#pragma unroll
    for (int rt = 0; rt < F32M_RTILES; rt++) wrow[rt] = w + (size_t)min(row0 + 16 * rt + r, d - 1) * n;
    f32x4 acc[F32M_RTILES][F32M_BTILES];
#pragma unroll
    for (int rt = 0; rt < F32M_RTILES; rt++)
#pragma unroll
        for (int t = 0; t < F32M_BTILES; t++) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nchunk = n / 64;
    for (int ch = wave; ch < nchunk; ch += F32M_WAVES) {
        const int k = 64 * ch + 16 * g;
        float wv[F32M_RTILES][16];
#pragma unroll
        for (int rt = 0; rt < F32M_RTILES; rt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = reinterpret_cast<const float4*>(wrow[rt] + k)[i];
                wv[rt][4 * i] = v.x;
                wv[rt][4 * i + 1] = v.y;
                wv[rt][4 * i + 2] = v.z;
                wv[rt][4 * i + 3] = v.w;
            }
#pragma unroll
        for (int t = 0; t < F32M_BTILES; t++) {
            if (t >= btiles) break;  // uniform
            const int bb = b0 + 16 * t + r;
            float xv[16];
            if (bb < batch) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 v = reinterpret_cast<const float4*>(x + (size_t)bb * n + k)[i];
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
            for (int rt = 0; rt < F32M_RTILES; rt++)
#pragma unroll
                for (int m = 0; m < 16; m++)
                    acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[rt][m], xv[m], acc[rt][t], 0, 0, 0);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int rt = 0; rt < F32M_RTILES; rt++)
#pragma unroll
            for (int t = 0; t < F32M_BTILES; t++)
                if (t < btiles) red[wave - 1][rt][t][lane] = acc[rt][t];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int rt = 0; rt < F32M_RTILES; rt++)
#pragma unroll
        for (int t = 0; t < F32M_BTILES; t++) {
            if (t >= btiles) break;
            f32x4 s = acc[rt][t];
#pragma unroll
            for (int v = 0; v < F32M_WAVES - 1; v++) s += red[v][rt][t][lane];
            const int bb = b0 + 16 * t + (lane & 15);
            if (bb >= batch) continue;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int row = row0 + 16 * rt + 4 * (lane >> 4) + j;
                if (row < d) out[(size_t)bb * d + row] = s[j];
            }
        }
}

}  // namespace

hipError_t launch_embed_rows(const float* table, const int32_t* tokens, float* x, int rows, int dim,
                             int vocab, int32_t* bad_tokens, float* ss, hipStream_t stream) {
    hipLaunchKernelGGL(embed_rows_kernel, dim3(rows), dim3(ROW_THREADS), 0, stream, table, tokens, x,
                       dim, vocab, bad_tokens, ss);
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm(float* x, const float* delta, const float* weight, float* out, int rows,
                              int dim, hipStream_t stream) {
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(rows), dim3(ROW_THREADS), 0, stream, x, delta, weight,
                       out, dim);
    return hipGetLastError();
}

hipError_t launch_gather_last_rows(const float* x, const float* ffn, const int32_t* row_off,
                                  const int32_t* len, float* last, int chunks, int dim,
                                  hipStream_t stream) {
    hipLaunchKernelGGL(gather_last_rows_kernel, dim3(chunks), dim3(ROW_THREADS), 0, stream, x, ffn,
                       row_off, len, last, dim);
    return hipGetLastError();
}

hipError_t launch_swiglu(float* hb, const float* hb2, size_t n, hipStream_t stream) {
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + ROW_THREADS - 1) / ROW_THREADS)),
                       dim3(ROW_THREADS), 0, stream, hb, hb2, n);
    return hipGetLastError();
}

namespace {
int f32_device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;
    }
    return cus[dev];
}

template <bool NORM, bool NT_W>
void launch_f32_flat_as(dim3 grid, dim3 block, size_t lds, hipStream_t stream, const float* w, const float* x,
                        float* out, int batch, int n, int d, const Q8Norm& nm) {
    switch (batch) {
        case 1: hipLaunchKernelGGL((f32_flat_kernel<1, NORM, NT_W>), grid, block, lds, stream, w, x, out, n, d, nm); break;
        case 2: hipLaunchKernelGGL((f32_flat_kernel<2, NORM, NT_W>), grid, block, lds, stream, w, x, out, n, d, nm); break;
        case 3: hipLaunchKernelGGL((f32_flat_kernel<3, NORM, NT_W>), grid, block, lds, stream, w, x, out, n, d, nm); break;
        default: hipLaunchKernelGGL((f32_flat_kernel<4, NORM, NT_W>), grid, block, lds, stream, w, x, out, n, d, nm); break;
    }
}

// f32_flat_kernel, one round of workgroups (2 per CU at up to 2 activation
// rows, whose registers allow it, else 1), if x and the sums fit 64 KiB of LDS.
template <bool NORM>
bool launch_f32_flat(const float* w, const float* x, float* out, int batch, int n, int d, const Q8Norm& nm,
                     hipStream_t stream) {
    const int groups_total = (d + 1) / 2;
    const int wgs = std::min(groups_total, (batch <= 2 ? 2 : 1) * f32_device_cus());
    const size_t rows_max = (size_t)((groups_total + wgs - 1) / wgs) * 2;
    const size_t lds = ((size_t)batch * n + rows_max * batch * F32F_WAVES + batch) * sizeof(float);
    if (lds > 64 * 1024) return false;  // the default dynamic LDS limit
    const dim3 grid((unsigned)wgs), block(64 * F32F_WAVES);
    if ((size_t)d * n * sizeof(float) >= F32F_NT_MIN_BYTES)
        launch_f32_flat_as<NORM, true>(grid, block, lds, stream, w, x, out, batch, n, d, nm);
    else
        launch_f32_flat_as<NORM, false>(grid, block, lds, stream, w, x, out, batch, n, d, nm);
    return true;
}
}  // namespace

hipError_t launch_f32_matmul(const float* w, const float* x, float* out, int batch, int n, int d,
                             hipStream_t stream) {
    if (n % 64 != 0) return hipErrorInvalidValue;
    if (batch <= 4 && batch * n <= F32F_X_MAX && launch_f32_flat<false>(w, x, out, batch, n, d, Q8Norm{}, stream))
        return hipGetLastError();
    if (batch <= 4) {
        const dim3 grid((unsigned)((d + 15) / 16)), block(64 * F32_WAVES);
        switch (batch) {
            case 1: hipLaunchKernelGGL(f32_gemv_kernel<1>, grid, block, 0, stream, w, x, out, n, d); break;
            case 2: hipLaunchKernelGGL(f32_gemv_kernel<2>, grid, block, 0, stream, w, x, out, n, d); break;
            case 3: hipLaunchKernelGGL(f32_gemv_kernel<3>, grid, block, 0, stream, w, x, out, n, d); break;
            default: hipLaunchKernelGGL(f32_gemv_kernel<4>, grid, block, 0, stream, w, x, out, n, d); break;
        }
        return hipGetLastError();
    }
    const unsigned by = (unsigned)((batch + 16 * F32M_BTILES - 1) / (16 * F32M_BTILES));
    if (batch > 16)
        hipLaunchKernelGGL(f32_matmul_mfma_kernel<2>, dim3((unsigned)((d + 31) / 32), by), dim3(64 * F32M_WAVES), 0,
                           stream, w, x, out, batch, n, d);
    else
        hipLaunchKernelGGL(f32_matmul_mfma_kernel<1>, dim3((unsigned)((d + 15) / 16), by), dim3(64 * F32M_WAVES), 0,
                           stream, w, x, out, batch, n, d);
    return hipGetLastError();
}

bool launch_f32_matmul_norm(const float* w, const float* x, const Q8Norm& nm, float* out, int batch, int n, int d,
                            hipStream_t stream) {
    if (n % 64 != 0 || batch > 4 || batch * n > F32F_X_MAX) return false;
    return launch_f32_flat<true>(w, x, out, batch, n, d, nm, stream);
}

}  // namespace nitro
