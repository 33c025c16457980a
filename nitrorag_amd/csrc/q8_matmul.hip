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
// Kernels, by activation rows and semantics (the launcher picks):
//  - last block only, any rows: q8_last_kernel on v_mfma_f32_16x16x4_f32
//    (fp32 in, fp32 accumulate), one wave per 16 activation rows.
//  - full rows, 1..4 rows: VALU dot products.  Rows of >= 2048 k take
//    q8_flat_kernel when the activations fit its LDS (batch x n <= 16384
//    floats), else q8_rowdot_kernel; q8_gemv_kernel covers short rows.
//  - full rows, more rows: q8_mma_kernel, the bf16 matrix cores at fp32
//    accuracy (x split into three exact bf16 parts), over the model's
//    tile-layout copy of the matrix when there is one (Q8Tiled) or the BlockQ8
//    rows otherwise; q8_matmul_kernel on v_mfma_f32_16x16x4_f32 under
//    NITRO_Q8_MMA=f32 or where the bf16 kernel's 32-bit offsets do not fit.
// Each kernel's comment gives its lane layout.
//
// A launch may cover a group of up to 3 matrices with the same input x and
// n (wq/wk/wv; w1/w3): a workgroup computes the same 16 rows of each member
// (members with fewer rows skip the upper tiles), and for the w1/w3 pair the
// epilogue applies SwiGLU, hb = silu(w1.x) * (w3.x) (src/model_q8.cpp:672-680),
// so the hidden activations are written once.
//
// The layer's rms_norm and residual adds live in these launches too:
//  - NORM (the wq/wk/wv and w1/w3 groups): x is the raw residual stream and
//    the input is rms_norm(x, weight) (src/model_q8.cpp:128-140): each x the
//    kernel loads becomes weight[k] * (inv * x[b][k]), inv = 1 / sqrtf(ss / n
//    + 1e-5), ss the sum of the row's partial sums of squares (written by
//    the launch that last changed x), added in a fixed order;
//  - RESID (wo, w2): the product is added into x in place and, per 16-row
//    output tile, the squares of each batch row's 16 new entries are summed
//    into one partial (tile p of row b at ss[p * ss_stride + b]);
//  - ROPE (wq/wk/wv): q and k rotated, q to its buffer, k and v to the pools.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "bf16_split.hpp"
#include "device_pool.hpp"

namespace nitro {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int Q8_BLOCK = 32;         // weights per block
constexpr int Q8_BLOCK_BYTES = 36;   // float scale + 32 int8
constexpr int Q8_WAVES = 4;
constexpr int Q8_MAX_BTILES = 4;     // batch tiles of 16 per launch row (batch <= 64 per grid.y)
constexpr int Q8_UNROLL = 4;         // 64-weight chunks whose loads a wave issues together

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

// load_slice without a branch: an invalid slice reads block 0 of the row
// (always in bounds) and gets scale 0, so every lane issues the same loads
// and the waits before use count exactly the loads that are needed.
__device__ __forceinline__ Q8Slice load_slice_always(const uint8_t* wrow, int blk, int half, bool valid) {
    const uint8_t* bp = wrow + (size_t)(valid ? blk : 0) * 36;
    const uint32_t* qp = reinterpret_cast<const uint32_t*>(bp + 4 + 16 * half);
    Q8Slice s{{qp[0], qp[1], qp[2], qp[3]}, *reinterpret_cast<const float*>(bp)};
    if (!valid) s.scale = 0.0f;
    return s;
}

__device__ __forceinline__ float sum_over_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Weight j (0..3) of a word of int8 weights, as a float.
__device__ __forceinline__ float q8_value(uint32_t w, int j) { return (float)(int)(int8_t)(w >> (8 * j)); }

__device__ __forceinline__ float dequant(uint32_t q4, int j, float scale) {
    return (float)(int)(int8_t)(q4 >> (8 * j)) * scale;
}

// Partials first, first + step, ... of batch row b, added in that order; the
// loads of 16 partials are issued before any is added (one round trip for a
// row of up to 16 * step partials).
__device__ __forceinline__ float partial_sum(const Q8Norm& nm, int b, int first, int step) {
    float s = 0.0f;
    for (int p0 = first; p0 < nm.nparts; p0 += 16 * step) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int p = p0 + i * step;
            v[i] = p < nm.nparts ? nm.ss[(size_t)p * nm.ss_stride + b] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) s += v[i];
    }
    return s;
}

// partial_sum with no branch around its loads: an index past the end rereads
// the last partial and adds 0 (same order of adds), so all L loads of a round
// go out together, behind any loads issued before.
template <int L>
__device__ __forceinline__ float partial_sum_unbranched(const Q8Norm& nm, int b, int first, int step) {
    float s = 0.0f;
    for (int p0 = first; p0 < nm.nparts; p0 += L * step) {
        float v[L];
#pragma unroll
        for (int i = 0; i < L; i++) v[i] = nm.ss[(size_t)min(p0 + i * step, nm.nparts - 1) * nm.ss_stride + b];
#pragma unroll
        for (int i = 0; i < L; i++) s += p0 + i * step < nm.nparts ? v[i] : 0.0f;
    }
    return s;
}

__device__ __forceinline__ float inv_rms(float ss, int n) { return 1.0f / sqrtf(ss / (float)n + 1e-5f); }

// Where batch row b's K/V goes and the position it rotates with.
struct RopeRow {
    int pos, page, in_page;
    bool page_ok;
};

__device__ __forceinline__ RopeRow rope_row(const Q8Rope& rp, int b) {
    const int w = b < rp.split ? 0 : 1;
    const int i = w ? b - rp.split : b;
    RopeRow r;
    r.pos = rp.pos[w][i];
    const int slot = rp.slot[w][i];
    r.page = slot >> 4;
    r.in_page = slot & 15;
    r.page_ok = r.page >= 0 && r.page < rp.num_pages;
    return r;
}

// (x, y) rotated by the angle of pair f of position pos: the reference's
// (x*fcr - y*fci, x*fci + y*fcr) (src/model_q8.cpp:600-612).
__device__ __forceinline__ float2 rotate_pair(const Q8Rope& rp, int pos, int feature, float x, float y) {
    const int f = (feature % rp.head_dim) >> 1;
    const float c = rp.freq_real[(size_t)pos * (rp.head_dim >> 1) + f];
    const float sn = rp.freq_imag[(size_t)pos * (rp.head_dim >> 1) + f];
    return make_float2(x * c - y * sn, x * sn + y * c);
}

}  // namespace

// Up to 3 matrices sharing x (same n); out[m] is [batch][d[m]]; wt[m] the
// same matrix in the tile layout (or null).
struct Q8Group {
    const uint8_t* w[3];
    float* out[3];
    int d[3];
    const uint8_t* wt[3];
};

namespace {

// The epilogue of one 16 x 16 output tile held as fp32 MFMA accumulators: lane
// l holds out^T[row0 + 4*(l/16) + j][bb] (j = 0..3) of each group member, bb
// = the tile's batch row l%16.  ROPE rotates q and k and appends k, v to the
// pools; RESID adds into x and writes the tile's sums of squares per batch
// row (partial `tile` of row bb; every lane must take part); SWIGLU or plain
// stores otherwise.
template <int NMAT, bool SWIGLU, bool RESID, bool ROPE>
__device__ __forceinline__ void store_mma_tile(const Q8Group& grp, const Q8Resid& resid, const Q8Rope& rope,
                                               const f32x4 (&s)[NMAT], int row0, int tile, int bb, int batch,
                                               int lane) {
    if constexpr (ROPE) {
        // q, k, v for features f0..f0+3 of row bb: two RoPE pairs
        if (bb >= batch) return;
        const RopeRow rr = rope_row(rope, bb);
        const int f0 = row0 + 4 * (lane >> 4);
        if (f0 < grp.d[0]) {
            const float2 a = rotate_pair(rope, rr.pos, f0, s[0][0], s[0][1]);
            const float2 c = rotate_pair(rope, rr.pos, f0 + 2, s[0][2], s[0][3]);
            *reinterpret_cast<float4*>(grp.out[0] + (size_t)bb * grp.d[0] + f0) = make_float4(a.x, a.y, c.x, c.y);
        }
        if (f0 < grp.d[1]) {
            if (rr.page_ok) {
                const size_t o = (size_t)rr.page * rope.page_stride + rope.layer_off +
                                 (size_t)rr.in_page * grp.d[1] + f0;
                const float2 a = rotate_pair(rope, rr.pos, f0, s[1][0], s[1][1]);
                const float2 c = rotate_pair(rope, rr.pos, f0 + 2, s[1][2], s[1][3]);
                *reinterpret_cast<float4*>(rope.k_pool + o) = make_float4(a.x, a.y, c.x, c.y);
                *reinterpret_cast<float4*>(rope.v_pool + o) = make_float4(s[2][0], s[2][1], s[2][2], s[2][3]);
            } else if (f0 == 0) {
                atomicAdd(rope.bad_pages, 1);  // once per row: the lane holding feature 0
            }
        }
    } else if constexpr (RESID) {
        // x[bb][row] += product; the squares of the tile's 16 new entries
        // of row bb are summed over the four lane groups (rows 4*(l/16) + j)
        float ssq = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = row0 + 4 * (lane >> 4) + j;
            if (bb < batch && row < grp.d[0]) {
                float* xe = grp.out[0] + (size_t)bb * grp.d[0] + row;
                const float v = *xe + s[0][j];
                *xe = v;
                ssq = fmaf(v, v, ssq);
            }
        }
        ssq = sum_over_rows(ssq);
        if (lane < 16 && bb < batch) resid.ss[(size_t)tile * resid.ss_stride + bb] = ssq;
    } else {
        if (bb >= batch) return;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = row0 + 4 * (lane >> 4) + j;
            if constexpr (SWIGLU) {
                if (row < grp.d[0]) {
                    float h = s[0][j];
                    h *= 1.0f / (1.0f + expf(-h));
                    grp.out[0][(size_t)bb * grp.d[0] + row] = h * s[1][j];
                }
            } else {
#pragma unroll
                for (int m = 0; m < NMAT; m++)
                    if (row < grp.d[m]) grp.out[m][(size_t)bb * grp.d[m] + row] = s[m][j];
            }
        }
    }
}

// fp32 matrix cores (v_mfma_f32_16x16x4_f32): a workgroup owns 16 output
// rows; out^T[16 rows][16 batch] += W[16 rows][4 k] . x^T[4 k][16 batch] per
// instruction.  Per 64-k chunk (two blocks), lane l = (r = l%16, g = l/16)
// loads the 16 int8 of row r in half g%2 of block 2*chunk + g/2 (one 16-byte
// run) and that block's scale; MFMA m (0..15) takes the lane's m-th weight, so
// the k-slot g of instruction m is k = (2*chunk + g/2)*32 + (g%2)*16 + m, and
// the B operand lane (c, g) holds x[c][that k] (16 contiguous floats per
// lane).  The four waves take chunks round-robin (U at a time, loads issued
// before use) and add their partial tiles through LDS.  Batches of more than
// 16 rows reuse the dequantised weights for every 16-row batch tile.
template <int NMAT, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
__global__ __launch_bounds__(64 * Q8_WAVES) void q8_matmul_kernel(Q8Group grp, const float* __restrict__ x,
                                                                   int batch, int n, Q8Norm nm, Q8Resid resid,
                                                                   Q8Rope rope) {
    constexpr int U = NMAT == 1 ? Q8_UNROLL : 2;  // chunks in flight per wave
    __shared__ f32x4 red[Q8_WAVES - 1][NMAT][Q8_MAX_BTILES][64];
    __shared__ float norm_s[NORM ? Q8_WAVES * 64 : 1];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int row0 = blockIdx.x * 16;
    const int b0 = blockIdx.y * 16 * Q8_MAX_BTILES;  // first batch row of this launch row
    const int btiles = min(Q8_MAX_BTILES, (batch - b0 + 15) / 16);
    const int nb = n / Q8_BLOCK;
    const int nchunk = (nb + 1) / 2;
    if constexpr (NORM) {
        // thread (row j = tid % 64, class c = tid / 64) adds partials c, c + 4, ...;
        // then row j's four class sums are added in order: norm_s[j] = inv_rms
        const int j = threadIdx.x & 63, c = threadIdx.x >> 6;
        norm_s[c * 64 + j] = b0 + j < batch ? partial_sum(nm, b0 + j, c, Q8_WAVES) : 0.0f;
        __syncthreads();
        float ss = 0.0f;
#pragma unroll
        for (int cc = 0; cc < Q8_WAVES; cc++) ss += norm_s[cc * 64 + lane];
        __syncthreads();
        if (wave == 0) norm_s[lane] = inv_rms(ss, n);
        __syncthreads();
    }
    const uint8_t* wrow[NMAT];
    bool act[NMAT];  // uniform: this tile has rows of member m
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        act[m] = row0 < grp.d[m];
        wrow[m] = grp.w[m] + (size_t)min(row0 + r, grp.d[m] - 1) * nb * Q8_BLOCK_BYTES;
    }

    f32x4 acc[NMAT][Q8_MAX_BTILES];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int t = 0; t < Q8_MAX_BTILES; t++) acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Wave w takes chunks (round*Q8_WAVES + w)*U + u.
    for (int base = wave * U; base < nchunk; base += Q8_WAVES * U) {
        Q8Slice sl[U][NMAT];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int blk = 2 * (base + u) + (g >> 1);
            const bool valid = base + u < nchunk && blk < nb;
#pragma unroll
            for (int m = 0; m < NMAT; m++) sl[u][m] = load_slice(wrow[m], blk, g & 1, valid && act[m]);
        }
        // Per batch tile, the x operands of all U chunks are loaded together
        // (one round trip), then the chunks' MFMAs run.
#pragma unroll
        for (int t = 0; t < Q8_MAX_BTILES; t++) {
            if (t >= btiles) break;  // uniform
            const int bb = b0 + t * 16 + r;  // batch row this lane feeds (B operand column)
            float xv[U][16];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int blk = 2 * (base + u) + (g >> 1);
                const bool valid = base + u < nchunk && blk < nb;
                if (valid && bb < batch) {
                    const int k0 = blk * Q8_BLOCK + 16 * (g & 1);
                    const float4* xp = reinterpret_cast<const float4*>(x + (size_t)bb * n + k0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float4 v = xp[i];
                        xv[u][4 * i] = v.x;
                        xv[u][4 * i + 1] = v.y;
                        xv[u][4 * i + 2] = v.z;
                        xv[u][4 * i + 3] = v.w;
                    }
                    if constexpr (NORM) {
                        const float inv = norm_s[t * 16 + r];
                        const float4* wp = reinterpret_cast<const float4*>(nm.weight + k0);
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float4 w = wp[i];
                            xv[u][4 * i] = w.x * (inv * xv[u][4 * i]);
                            xv[u][4 * i + 1] = w.y * (inv * xv[u][4 * i + 1]);
                            xv[u][4 * i + 2] = w.z * (inv * xv[u][4 * i + 2]);
                            xv[u][4 * i + 3] = w.w * (inv * xv[u][4 * i + 3]);
                        }
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < 16; q++) xv[u][q] = 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (base + u >= nchunk) break;  // uniform
#pragma unroll
                for (int m = 0; m < NMAT; m++) {
                    if (!act[m]) continue;  // uniform
                    float wv[16];
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        wv[jj] = dequant(sl[u][m].q[0], jj, sl[u][m].scale);
                        wv[4 + jj] = dequant(sl[u][m].q[1], jj, sl[u][m].scale);
                        wv[8 + jj] = dequant(sl[u][m].q[2], jj, sl[u][m].scale);
                        wv[12 + jj] = dequant(sl[u][m].q[3], jj, sl[u][m].scale);
                    }
#pragma unroll
                    for (int q = 0; q < 16; q++)
                        acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[q], xv[u][q], acc[m][t], 0, 0, 0);
                }
            }
        }
    }

    // Sum the four waves' partial tiles; wave 0 writes.  Lane l holds
    // out^T[row0 + 4*(l/16) + j][b0 + 16t + l%16], j = 0..3.
    if (wave > 0) {
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int t = 0; t < Q8_MAX_BTILES; t++)
                if (t < btiles) red[wave - 1][m][t][lane] = acc[m][t];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int t = 0; t < Q8_MAX_BTILES; t++) {
        if (t >= btiles) break;  // uniform
        f32x4 s[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            s[m] = acc[m][t];
#pragma unroll
            for (int v = 0; v < Q8_WAVES - 1; v++) s[m] += red[v][m][t][lane];
        }
        store_mma_tile<NMAT, SWIGLU, RESID, ROPE>(grp, resid, rope, s, row0, blockIdx.x, b0 + t * 16 + (lane & 15),
                                                  batch, lane);
    }
}

// matmul_bulk (src/model_q8.cpp:382-420: each output row keeps only its last
// 32-column block, the block loop storing over the previous block's sum), for
// any number of activation rows.  A workgroup covers 16 output rows (of each
// group member) and 64 batch rows, one wave per batch tile of 16.  Every load
// a wave needs goes out at its start, in one round trip: the rows' last
// blocks (lane (r, g): weights 8g..8g+7 of row row0 + r and the row's scale),
// x of batch row 16t + r at the same 8 k, and with the norm folded in that
// row's norm weights and rms partials (lane group g adding partials g, g + 4,
// ..., the four groups then summed by permutes).  Eight fp32 MFMAs per member
// cover the block (MFMA j takes k = 8g + j in k-slot g), and each wave runs
// the epilogue on its own tile: no reduction across waves, no barrier.  (As a
// mode of the full-row kernels, q8_matmul_kernel ran the block on one wave of
// four, half its 16 MFMAs on zeros, behind the partials' round trip and three
// barriers, and q8_gemv_kernel staged the block's x through LDS: continuous
// batching at 32 users took 22.8-23.7 ms per run then, 18.8-20.0 now.)
template <int NMAT, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
__global__ __launch_bounds__(64 * Q8_WAVES) void q8_last_kernel(Q8Group grp, const float* __restrict__ x, int batch,
                                                                 int n, Q8Norm nm, Q8Resid resid, Q8Rope rope) {
    static_assert(Q8_MAX_BTILES == Q8_WAVES, "the launch grid gives each launch row one wave per batch tile");
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int row0 = blockIdx.x * 16;
    const int t = blockIdx.y * Q8_WAVES + wave;  // this wave's batch tile
    if (t * 16 >= batch) return;                 // wave-uniform; the kernel has no barrier
    const int nb = n / Q8_BLOCK;
    const int k0 = (nb - 1) * Q8_BLOCK + 8 * g;  // the lane's 8 k of the last block
    const int bx = min(t * 16 + r, batch - 1);   // the batch row it feeds (clamped: never stored)
    uint32_t q[NMAT][2];
    float sc[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const uint8_t* bp = grp.w[m] + ((size_t)min(row0 + r, grp.d[m] - 1) * nb + nb - 1) * Q8_BLOCK_BYTES;
        const uint32_t* qp = reinterpret_cast<const uint32_t*>(bp + 4 + 8 * g);
        q[m][0] = qp[0];
        q[m][1] = qp[1];
        sc[m] = *reinterpret_cast<const float*>(bp);
    }
    const float4* xp = reinterpret_cast<const float4*>(x + (size_t)bx * n + k0);
    const float4 xa = xp[0], xb = xp[1];
    float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    if constexpr (NORM) {
        const float4* wp = reinterpret_cast<const float4*>(nm.weight + k0);
        const float4 wa = wp[0], wb = wp[1];
        const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
        const float inv = inv_rms(sum_over_rows(partial_sum(nm, bx, g, 4)), n);
#pragma unroll
        for (int j = 0; j < 8; j++) xv[j] = wv[j] * (inv * xv[j]);
    }
    // RoPE: the lane's output features f0..f0+3 (two pairs of one head) of
    // batch row bx.  Its position and slot, and the pairs' cos / sin, load
    // here too, so their two dependent round trips overlap the products'
    // loads (the wq/wk/wv launch at 32 rows: 4.47 -> 4.30 us).
    const int f0 = row0 + 4 * g;
    RopeRow rr{};
    float rc[2] = {0.f, 0.f}, rs[2] = {0.f, 0.f};
    if constexpr (ROPE) {
        rr = rope_row(rope, bx);
        const size_t fi = (size_t)rr.pos * (rope.head_dim >> 1) + ((f0 % rope.head_dim) >> 1);
        rc[0] = rope.freq_real[fi];
        rs[0] = rope.freq_imag[fi];
        rc[1] = rope.freq_real[fi + 1];
        rs[1] = rope.freq_imag[fi + 1];
    }
    f32x4 s[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        s[m] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (row0 >= grp.d[m]) continue;  // uniform: no rows of member m in this tile
#pragma unroll
        for (int j = 0; j < 8; j++)
            s[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(dequant(q[m][j >> 2], j & 3, sc[m]), xv[j], s[m], 0, 0, 0);
    }
    if constexpr (ROPE) {
        // store_mma_tile's RoPE epilogue on the prefetched angles
        // (rotate_pair's (x*c - y*sn, x*sn + y*c))
        const int bb = t * 16 + r;
        if (bb >= batch) return;
        auto rot = [&](int p, float u, float v) { return make_float2(u * rc[p] - v * rs[p], u * rs[p] + v * rc[p]); };
        if (f0 < grp.d[0]) {
            const float2 a = rot(0, s[0][0], s[0][1]);
            const float2 c = rot(1, s[0][2], s[0][3]);
            *reinterpret_cast<float4*>(grp.out[0] + (size_t)bb * grp.d[0] + f0) = make_float4(a.x, a.y, c.x, c.y);
        }
        if (f0 < grp.d[1]) {
            if (rr.page_ok) {
                const size_t o = (size_t)rr.page * rope.page_stride + rope.layer_off +
                                 (size_t)rr.in_page * grp.d[1] + f0;
                const float2 a = rot(0, s[1][0], s[1][1]);
                const float2 c = rot(1, s[1][2], s[1][3]);
                *reinterpret_cast<float4*>(rope.k_pool + o) = make_float4(a.x, a.y, c.x, c.y);
                *reinterpret_cast<float4*>(rope.v_pool + o) = make_float4(s[2][0], s[2][1], s[2][2], s[2][3]);
            } else if (f0 == 0) {
                atomicAdd(rope.bad_pages, 1);  // once per row: the lane holding feature 0
            }
        }
    } else {
        store_mma_tile<NMAT, SWIGLU, RESID, ROPE>(grp, resid, rope, s, row0, blockIdx.x, t * 16 + r, batch, lane);
    }
}

// Batches of 1..NB rows on the VALU: lane (r, g) dots its 16 weights of row
// row0 + r with x[b] at the same 16 k for every b.  A workgroup of
// GEMV_WAVES waves owns 16 rows (of each group member); per slab of
// GEMV_WAVES*U chunks (2048 k for one matrix) each wave first issues the
// weight loads of its U chunks, then the workgroup stages the slab of x in
// LDS (lanes of a lane group read the same x, which LDS broadcasts; NORM
// applies rms_norm while staging), and then the waves compute.  The 4 lane
// groups are summed with row-swap permutes and the waves through LDS in a
// fixed order (results are repeatable bit for bit).
constexpr int GEMV_WAVES = 8;

#ifndef NITRO_GEMV_UNROLL
#define NITRO_GEMV_UNROLL 8
#endif
template <int NB, int NMAT, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
__global__ __launch_bounds__(64 * GEMV_WAVES) void q8_gemv_kernel(Q8Group grp, const float* __restrict__ x,
                                                                   int n, Q8Norm nm, Q8Resid resid, Q8Rope rope) {
    // chunks in flight per wave: a slab covers 4096 k of one matrix (2048 of a group)
    constexpr int U = NMAT == 1 ? NITRO_GEMV_UNROLL : NITRO_GEMV_UNROLL / 2;
    constexpr int SLAB = GEMV_WAVES * U * 64;     // k per slab
    __shared__ __attribute__((aligned(16))) float xs[NB][SLAB];
    __shared__ float red[GEMV_WAVES][NMAT][NB][16];
    __shared__ float inv_s[NB];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int row0 = blockIdx.x * 16;
    const int nb = n / Q8_BLOCK;
    const int nchunk = (nb + 1) / 2;
    if constexpr (NORM) {
        // wave b < NB: lane i adds row b's partials i, i + 64, ...; then the
        // 64 lane sums are added (ordered before use by the barrier ahead of
        // the first slab's staging)
        if (wave < NB) {
            float v = partial_sum(nm, wave, lane, 64);
#pragma unroll
            for (int msk = 32; msk > 0; msk >>= 1) v += __shfl_xor(v, msk);
            if (lane == 0) inv_s[wave] = inv_rms(v, n);
        }
    }
    const uint8_t* wrow[NMAT];
    bool act[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        act[m] = row0 < grp.d[m];
        wrow[m] = grp.w[m] + (size_t)min(row0 + r, grp.d[m] - 1) * nb * Q8_BLOCK_BYTES;
    }

    float acc[NMAT][NB];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[m][b] = 0.0f;

    for (int slab = 0; slab < n; slab += SLAB) {
        const int c0 = slab / 64 + wave * U;  // this wave's first chunk
        Q8Slice sl[U][NMAT];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int blk = 2 * (c0 + u) + (g >> 1);
            const bool valid = c0 + u < nchunk && blk < nb;
#pragma unroll
            for (int m = 0; m < NMAT; m++) sl[u][m] = load_slice(wrow[m], blk, g & 1, valid && act[m]);
        }
        const int slab_len = min(SLAB, n - slab);  // multiple of 32
        __syncthreads();  // previous slab's x reads are done
#pragma unroll
        for (int b = 0; b < NB; b++)
            for (int f = threadIdx.x; f < slab_len / 4; f += 64 * GEMV_WAVES) {
                float4 v = reinterpret_cast<const float4*>(x + (size_t)b * n + slab)[f];
                if constexpr (NORM) {
                    const float inv = inv_s[b];
                    const float4 w = reinterpret_cast<const float4*>(nm.weight + slab)[f];
                    v = make_float4(w.x * (inv * v.x), w.y * (inv * v.y), w.z * (inv * v.z), w.w * (inv * v.w));
                }
                *reinterpret_cast<float4*>(&xs[b][4 * f]) = v;
            }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int blk = 2 * (c0 + u) + (g >> 1);
            const bool valid = c0 + u < nchunk && blk < nb;
            if (!valid) continue;  // no cross-lane work inside the chunk loop
            const int kl = blk * Q8_BLOCK + 16 * (g & 1) - slab;  // k within the slab
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                if (!act[m]) continue;
                float wv[16];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    wv[jj] = dequant(sl[u][m].q[0], jj, sl[u][m].scale);
                    wv[4 + jj] = dequant(sl[u][m].q[1], jj, sl[u][m].scale);
                    wv[8 + jj] = dequant(sl[u][m].q[2], jj, sl[u][m].scale);
                    wv[12 + jj] = dequant(sl[u][m].q[3], jj, sl[u][m].scale);
                }
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const float4* xp = reinterpret_cast<const float4*>(&xs[b][kl]);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 v = xp[q];
                        acc[m][b] = fmaf(wv[4 * q], v.x, acc[m][b]);
                        acc[m][b] = fmaf(wv[4 * q + 1], v.y, acc[m][b]);
                        acc[m][b] = fmaf(wv[4 * q + 2], v.z, acc[m][b]);
                        acc[m][b] = fmaf(wv[4 * q + 3], v.w, acc[m][b]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[m][b] = sum_over_rows(acc[m][b]);  // lanes r, r+16, r+32, r+48
    if (g == 0) {
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int b = 0; b < NB; b++) red[wave][m][b][r] = acc[m][b];
    }
    __syncthreads();
    if (threadIdx.x >= NB * 16) return;
    const int b = threadIdx.x / 16, rr = threadIdx.x % 16;
    const int row = row0 + rr;
    float sum[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        sum[m] = 0.0f;
#pragma unroll
        for (int v = 0; v < GEMV_WAVES; v++) sum[m] += red[v][m][b][rr];
    }
    if constexpr (ROPE) {
        // RoPE pairs are features (row, row ^ 1): adjacent lanes of the group
        const float q_o = __shfl_xor(sum[0], 1), k_o = __shfl_xor(sum[1], 1);
        const RopeRow rp = rope_row(rope, b);
        const bool odd = rr & 1;
        const int fe = row & ~1;
        const float2 qr = rotate_pair(rope, rp.pos, fe, odd ? q_o : sum[0], odd ? sum[0] : q_o);
        const float2 kr = rotate_pair(rope, rp.pos, fe, odd ? k_o : sum[1], odd ? sum[1] : k_o);
        if (row < grp.d[0]) grp.out[0][(size_t)b * grp.d[0] + row] = odd ? qr.y : qr.x;
        if (row < grp.d[1]) {
            if (rp.page_ok) {
                const size_t o = (size_t)rp.page * rope.page_stride + rope.layer_off +
                                 (size_t)rp.in_page * grp.d[1] + row;
                rope.k_pool[o] = odd ? kr.y : kr.x;
                rope.v_pool[o] = sum[2];
            } else if (row == 0) {
                atomicAdd(rope.bad_pages, 1);  // once per row
            }
        }
        return;
    }
    if constexpr (RESID) {
        // x[b][row] += product; the 16 lanes of batch row b add their squares
        float ssq = 0.0f;
        if (row < grp.d[0]) {
            float* xe = grp.out[0] + (size_t)b * grp.d[0] + row;
            const float v = *xe + sum[0];
            *xe = v;
            ssq = v * v;
        }
#pragma unroll
        for (int msk = 8; msk > 0; msk >>= 1) ssq += __shfl_xor(ssq, msk, 16);
        if (rr == 0) resid.ss[(size_t)blockIdx.x * resid.ss_stride + b] = ssq;
    } else if constexpr (SWIGLU) {
        if (row < grp.d[0]) {
            float h = sum[0];
            h *= 1.0f / (1.0f + expf(-h));
            grp.out[0][(size_t)b * grp.d[0] + row] = h * sum[1];
        }
    } else {
#pragma unroll
        for (int m = 0; m < NMAT; m++)
            if (row < grp.d[m]) grp.out[m][(size_t)b * grp.d[m] + row] = sum[m];
    }
}

// The epilogue of one output element, out[b][row] of each group member, for
// kernels that hold finished sums one element per thread: `pair` holds the
// q and k sums of row row ^ 1 (RoPE pairs).  RESID: the 16 threads of rows
// 16p..16p+15 of batch row b must be 16 consecutive lanes (ordered by row)
// and call this together; they add their squares into partial p of row b.
template <int NMAT, bool SWIGLU, bool RESID, bool ROPE>
__device__ __forceinline__ void store_row_sums(const Q8Group& grp, const Q8Resid& resid, const Q8Rope& rope, int b,
                                               int row, const float (&sum)[NMAT], const float (&pair)[2]) {
    if constexpr (ROPE) {
        const RopeRow rp = rope_row(rope, b);
        const bool odd = row & 1;
        const int fe = row & ~1;
        const float2 qr = rotate_pair(rope, rp.pos, fe, odd ? pair[0] : sum[0], odd ? sum[0] : pair[0]);
        const float2 kr = rotate_pair(rope, rp.pos, fe, odd ? pair[1] : sum[1], odd ? sum[1] : pair[1]);
        if (row < grp.d[0]) grp.out[0][(size_t)b * grp.d[0] + row] = odd ? qr.y : qr.x;
        if (row < grp.d[1]) {
            if (rp.page_ok) {
                const size_t o = (size_t)rp.page * rope.page_stride + rope.layer_off +
                                 (size_t)rp.in_page * grp.d[1] + row;
                rope.k_pool[o] = odd ? kr.y : kr.x;
                rope.v_pool[o] = sum[2];
            } else if (row == 0) {
                atomicAdd(rope.bad_pages, 1);  // once per row
            }
        }
    } else if constexpr (RESID) {
        // x[b][row] += product; the 16 threads of the row group add their squares
        float ssq = 0.0f;
        if (row < grp.d[0]) {
            float* xe = grp.out[0] + (size_t)b * grp.d[0] + row;
            const float v = *xe + sum[0];
            *xe = v;
            ssq = v * v;
        }
#pragma unroll
        for (int msk = 8; msk > 0; msk >>= 1) ssq += __shfl_xor(ssq, msk, 16);
        if ((row & 15) == 0 && row < grp.d[0]) resid.ss[(size_t)(row >> 4) * resid.ss_stride + b] = ssq;
    } else if constexpr (SWIGLU) {
        if (row < grp.d[0]) {
            float h = sum[0];
            h *= 1.0f / (1.0f + expf(-h));
            grp.out[0][(size_t)b * grp.d[0] + row] = h * sum[1];
        }
    } else {
#pragma unroll
        for (int m = 0; m < NMAT; m++)
            if (row < grp.d[m]) grp.out[m][(size_t)b * grp.d[m] + row] = sum[m];
    }
}

// Batches of 1..NB rows over long rows (full-row products, n >= 2048),
// weights streamed row by row.  A tile is 16R output rows: four row sets of
// four row groups of R rows.  A wave owns one row group of each set and half
// of the k range (chunks of 1024 k = 32 blocks, the two halves interleaved);
// lane l takes half l%2 of block 32*chunk + l/2 of each row, so one load
// instruction covers 32 consecutive blocks of a row (1152 contiguous bytes).
// A wave's work items (row set, chunk) run in order across the tile and on
// into its next tile (workgroups loop over tiles when the tiles outnumber
// ROWDOT_MAX_GROUPS), each item's weights loaded while the previous item is
// used, in two register sets that alternate.  x (with rms_norm)
// is read per item.  After a row set's last chunk the 64 lanes of each row
// are summed with a fixed butterfly into LDS; at the tile's end the two k
// halves are added in a fixed order and the epilogue (SwiGLU, RoPE + K/V
// append, residual) runs on the sums in LDS.
template <int NB, int NMAT>
constexpr int rowdot_rows() {
    return NMAT == 1 ? 4 : NMAT == 2 ? 2 : (NB <= 2 ? 2 : 1);
}
constexpr int ROWDOT_SETS = 1;

template <int NB, int NMAT, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
__global__ __launch_bounds__(512) void q8_rowdot_kernel(Q8Group grp, const float* __restrict__ x, int n,
                                                         int ntiles, Q8Norm nm, Q8Resid resid, Q8Rope rope) {
    constexpr int R = rowdot_rows<NB, NMAT>();
    constexpr int TROWS = ROWDOT_SETS * 4 * R;  // output rows per tile
    __shared__ float red[2][NMAT][TROWS][NB];
    __shared__ float inv_s[NB];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kh = wave & 1;   // k half
    const int rg = wave >> 1;  // row group within each set
    const int nb = n / Q8_BLOCK;
    const int nchunks = (nb + 31) / 32;
    const int per_set = (nchunks - kh + 1) / 2;  // chunks kh, kh + 2, ... (>= 1: n >= 2048)
    const int items = ROWDOT_SETS * per_set;
    // rows of item e of `tile`; e == items is the first item of the next tile
    auto item_rows = [&](int tile, int e, int& row_base, int& c) {
        if (e >= items) {
            tile += gridDim.x;
            e = 0;
        }
        const int set = e / per_set;
        c = kh + 2 * (e - set * per_set);
        row_base = tile < ntiles ? tile * TROWS + (set * 4 + rg) * R : INT32_MAX / 2;
    };
    auto load_item = [&](Q8Slice (&sl)[NMAT][R], int tile, int e) {
        int row_base, c;
        item_rows(tile, e, row_base, c);
        const int blk = 32 * c + (lane >> 1);
        const bool valid = blk < nb;
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = row_base + r;
                const uint8_t* wr = grp.w[m] + (size_t)min(row, grp.d[m] - 1) * nb * Q8_BLOCK_BYTES;
                sl[m][r] = load_slice_always(wr, blk, lane & 1, valid && row < grp.d[m]);
            }
    };
    auto load_x = [&](float (&xv)[NB][16], int e) {
        const int set = e / per_set;
        const int c = kh + 2 * (e - set * per_set);
        const int blk = 32 * c + (lane >> 1);
        // an invalid lane reads x[b][0..16) (in bounds); its weights are 0
        const int k0 = blk < nb ? blk * Q8_BLOCK + 16 * (lane & 1) : 0;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float4* xp = reinterpret_cast<const float4*>(x + (size_t)b * n + k0);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 v = xp[q];
                xv[b][4 * q] = v.x;
                xv[b][4 * q + 1] = v.y;
                xv[b][4 * q + 2] = v.z;
                xv[b][4 * q + 3] = v.w;
            }
            if constexpr (NORM) {
                const float inv = inv_s[b];
                const float4* wp = reinterpret_cast<const float4*>(nm.weight + k0);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 w = wp[q];
                    xv[b][4 * q] = w.x * (inv * xv[b][4 * q]);
                    xv[b][4 * q + 1] = w.y * (inv * xv[b][4 * q + 1]);
                    xv[b][4 * q + 2] = w.z * (inv * xv[b][4 * q + 2]);
                    xv[b][4 * q + 3] = w.w * (inv * xv[b][4 * q + 3]);
                }
            }
        }
    };
    float acc[NMAT][R][NB];
    auto clear = [&] {
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int b = 0; b < NB; b++) acc[m][r][b] = 0.0f;
    };
    // x of item e, then the next item's weights into `next`, then e's products
    // with `now`; after a row set's last chunk, its row sums go to LDS.
    auto step = [&](const Q8Slice (&now)[NMAT][R], Q8Slice (&next)[NMAT][R], int tile, int e) {
        float xv[NB][16];
        load_x(xv, e);
        load_item(next, tile, e + 1);
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                float wv[16];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    wv[jj] = dequant(now[m][r].q[0], jj, now[m][r].scale);
                    wv[4 + jj] = dequant(now[m][r].q[1], jj, now[m][r].scale);
                    wv[8 + jj] = dequant(now[m][r].q[2], jj, now[m][r].scale);
                    wv[12 + jj] = dequant(now[m][r].q[3], jj, now[m][r].scale);
                }
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int q = 0; q < 16; q++) acc[m][r][b] = fmaf(wv[q], xv[b][q], acc[m][r][b]);
            }
        const int set = e / per_set;
        if (e - set * per_set == per_set - 1) {  // the set's last chunk (wave-uniform)
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        float v = acc[m][r][b];
#pragma unroll
                        for (int msk = 32; msk > 0; msk >>= 1) v += __shfl_xor(v, msk);
                        if (lane == 0) red[kh][m][(set * 4 + rg) * R + r][b] = v;
                    }
            clear();
        }
    };
    Q8Slice sa[NMAT][R], sb[NMAT][R];
    load_item(sa, blockIdx.x, 0);
    if constexpr (NORM) {
        // wave b < NB adds row b's partials (lane i takes i, i + 64, ...)
        if (wave < NB) {
            float v = partial_sum(nm, wave, lane, 64);
#pragma unroll
            for (int msk = 32; msk > 0; msk >>= 1) v += __shfl_xor(v, msk);
            if (lane == 0) inv_s[wave] = inv_rms(v, n);
        }
        __syncthreads();
    }
    clear();
    // Items alternate between the two register sets; a tile with an odd item
    // count hands the next tile's first item over in the other set.
    auto run_tile = [&](auto& first, auto& second, int tile) {
        int e = 0;
        for (; e + 1 < items; e += 2) {
            step(first, second, tile, e);
            step(second, first, tile, e + 1);
        }
        if (e < items) step(first, second, tile, e);
    };
    bool flipped = false;
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        if (!flipped)
            run_tile(sa, sb, tile);
        else
            run_tile(sb, sa, tile);
        flipped ^= (items & 1) != 0;
        __syncthreads();
        for (int t = threadIdx.x; t < NB * TROWS; t += 512) {
            const int b = t / TROWS, i = t % TROWS;
            const int row = tile * TROWS + i;
            float sum[NMAT], pair[2] = {0.0f, 0.0f};
#pragma unroll
            for (int m = 0; m < NMAT; m++) sum[m] = red[0][m][i][b] + red[1][m][i][b];
            if constexpr (ROPE) {
                // RoPE pairs are rows (i, i ^ 1) of the tile
                pair[0] = red[0][0][i ^ 1][b] + red[1][0][i ^ 1][b];
                pair[1] = red[0][1][i ^ 1][b] + red[1][1][i ^ 1][b];
            }
            static_assert(!RESID || TROWS % 16 == 0, "residual partials are per 16 rows");
            store_row_sums<NMAT, SWIGLU, RESID, ROPE>(grp, resid, rope, b, row, sum, pair);
        }
        __syncthreads();  // red is reused by the next tile
    }
}

// The slice of block blk (in range) with no test on the loaded values: a
// select on them would make the wave wait for these loads where they are
// issued.  Lanes past the row are masked through their activations.
__device__ __forceinline__ Q8Slice load_slice_raw(const uint8_t* wrow, int blk, int half) {
    const uint8_t* bp = wrow + (size_t)blk * Q8_BLOCK_BYTES;
    const uint32_t* qp = reinterpret_cast<const uint32_t*>(bp + 4 + 16 * half);
    return Q8Slice{{qp[0], qp[1], qp[2], qp[3]}, *reinterpret_cast<const float*>(bp)};
}

// Batches of 1..NB rows over long rows (n >= 2048) whose activations fit LDS
// (NB * n <= flat_x_max floats).  x is staged in LDS once per workgroup
// (times the norm weights when NORM: rms_norm's 1/rms is one scalar per
// activation row, applied to the row sums in the epilogue, so staging x
// waits on no reduction; the reference scales x first, the two agree to fp32
// rounding), so a wave's only loads from memory in its loop are
// weights: x reads wait on the LDS counter, and the next item's weights stay
// in flight while the current item is used.  Persistent workgroups own
// balanced ranges of row units (16 rows with the residual epilogue, whose
// sums of squares are per 16-row tile; 2 rows otherwise, so RoPE pairs stay
// together).  Items are (group of FLAT_R rows, 1024-k chunk); the
// workgroup's items are split between its waves in contiguous runs.  Lane l
// reads half l%2 of block 32*chunk + l/2 of each row (1152 contiguous bytes
// per row and load instruction).  A block's products are summed, then scaled
// (sum_k q*x times the block's scale; the reference scales each weight
// first, src/model_q8.cpp:106-112, and the two agree to fp32 rounding).  At
// a group's last chunk, or the end
// of the wave's run, the 64 lanes of each row are summed with a fixed
// butterfly into the wave's slot in LDS; the epilogue adds the slots in wave
// order, so results do not depend on timing.
constexpr int FLAT_R = 2;              // rows per item

// Staged activations (NB * n floats) and LDS per workgroup at most: 64 KiB of
// x and 80 KiB in all, two workgroups per CU; with the residual epilogue, one
// 16-wave workgroup per CU (its registers allow no second), so 156 KiB of x
// and 160 KiB in all (rows of 11008 k at 2-3 activation rows).
template <bool RESID>
constexpr int flat_x_max() {
    return RESID ? 39936 : 16384;
}
template <bool RESID>
constexpr int flat_lds_max() {
    return RESID ? 160 * 1024 : 80 * 1024;
}

template <bool RESID>
constexpr int flat_unit_rows() {
    return RESID ? 16 : 2;
}
// Waves per workgroup: 16 with the residual epilogue, whose 16-row units
// leave fewer workgroups (256 for a 4096-row matrix), 8 otherwise.
template <bool RESID>
constexpr int flat_waves() {
    return RESID ? 16 : 8;
}

template <int NB, int NMAT, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
__global__ __launch_bounds__(64 * flat_waves<RESID>()) void q8_flat_kernel(Q8Group grp, const float* __restrict__ x,
                                                                           int n, int dmax, Q8Norm nm, Q8Resid resid,
                                                                           Q8Rope rope) {
    constexpr int W = flat_waves<RESID>(), NT = 64 * W, R = FLAT_R;
    constexpr int UG = flat_unit_rows<RESID>();
    // float4 of x per thread at most (rounded up: the last round may be partial)
    constexpr int XV = (flat_x_max<RESID>() / 4 + NT - 1) / NT;
    static_assert(flat_x_max<RESID>() % 4 == 0 && XV * 4 * NT >= flat_x_max<RESID>(),
                  "the staging loop must cover every float of x the launcher admits");
    extern __shared__ __attribute__((aligned(16))) float flat_lds[];  // float4 access: 16-byte base
    __shared__ float inv_s[NB];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nb = n / Q8_BLOCK;
    const int nch = (nb + 31) / 32;
    const int units = (dmax + UG - 1) / UG;
    const int u0 = (int)((long long)units * blockIdx.x / gridDim.x);
    const int u1 = (int)((long long)units * (blockIdx.x + 1) / gridDim.x);
    const int row0 = u0 * UG, rows = (u1 - u0) * UG;  // rows past dmax are computed, never stored
    const int items = rows / R * nch;
    const int i0 = items * wave / W, i1 = items * (wave + 1) / W;
    float* xs = flat_lds;          // [NB][n]
    float* red = flat_lds + NB * n;  // [rows][NMAT][NB][W]
    const size_t rowbytes = (size_t)nb * Q8_BLOCK_BYTES;

    // item i of the run -> local group g and chunk c (i clamped into the run,
    // so a wave with no items still loads in-range weights, never used)
    auto load_item = [&](Q8Slice (&sl)[NMAT][R], int i) {
        i = max(min(i, i1 - 1), 0);
        const int g = i / nch, c = i - g * nch;
        const int blk = 32 * c + (lane >> 1);
        const int bk = blk < nb ? blk : 0;  // a lane past the row reads block 0; its x are 0
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = min(row0 + g * R + r, grp.d[m] - 1);
                sl[m][r] = load_slice_raw(grp.w[m] + (size_t)row * rowbytes, bk, lane & 1);
            }
    };
    // The prologue's loads go out in the order they are needed: the first
    // XE float4 of x per thread (and of the norm weights; all of x for one
    // row of 4096 at 8 waves), the first PE rms partials per lane (all of
    // them for n <= 4096), then the first item's weights.  Loads complete in
    // order, so the waits for those x and partials do not wait for the
    // weights, which stay in flight while x is staged.  (Issued before them,
    // the weights were waited for with them; holding all of x early takes
    // too many registers.)  A float4 index past the end is clamped to the
    // last one, whose value its threads store again.
    constexpr int XE = XV < 2 ? XV : 2, PE = 4;
    const int total = NB * n / 4, nv = (total + NT - 1) / NT;  // uniform
    float4 xr[XV], wr[XV];
    auto load_x = [&](int v) {
        const int t = min((int)threadIdx.x + v * NT, total - 1);
        xr[v] = reinterpret_cast<const float4*>(x)[t];
        if constexpr (NORM) wr[v] = reinterpret_cast<const float4*>(nm.weight)[t % (n / 4)];
    };
#pragma unroll
    for (int v = 0; v < XE; v++)
        if (v < nv) load_x(v);
    // rms partials of batch row b = wave < NB, lane i taking partials i,
    // i + 64, ... in order (every wave loads, the others a clamped row,
    // unused)
    float pv[PE];
    if constexpr (NORM) {
        const int pb = min(wave, NB - 1);
#pragma unroll
        for (int i = 0; i < PE; i++) pv[i] = nm.ss[(size_t)min(lane + i * 64, nm.nparts - 1) * nm.ss_stride + pb];
    }
    Q8Slice sa[NMAT][R], sb[NMAT][R];
    // With the norm folded in, a workgroup is alone on its CU (its LDS), so
    // at one activation row the second item also goes out here, into
    // registers the loop would hold anyway: two items in flight while x is
    // staged, one from then on.  (7B step at B=1: 2.376 -> 2.362 ms; at B=2
    // the same was 1.2% slower.)
    constexpr bool EARLY2 = NORM && NB == 1;
    __builtin_amdgcn_sched_barrier(0);  // (left free, the scheduler puts the partials last)
    load_item(sa, i0);                  // in flight while x is staged
    if constexpr (EARLY2) load_item(sb, i0 + 1);
    __builtin_amdgcn_sched_barrier(0);
    {
        // the rest of x, then x -> LDS (times the norm weights when NORM; the
        // row's rms factor, a scalar per batch row, scales the row sums in
        // the epilogue, so staging x waits on no reduction)
#pragma unroll
        for (int v = XE; v < XV; v++)
            if (v < nv) load_x(v);
#pragma unroll
        for (int v = 0; v < XV; v++)
            if (v < nv) {
                const int t = min((int)threadIdx.x + v * NT, total - 1);
                float4 o = xr[v];
                if constexpr (NORM) o = make_float4(wr[v].x * o.x, wr[v].y * o.y, wr[v].z * o.z, wr[v].w * o.w);
                reinterpret_cast<float4*>(xs)[t] = o;
            }
    }
    for (int t = threadIdx.x; t < rows * NMAT * NB * W; t += NT) red[t] = 0.0f;
    __syncthreads();

    float acc[NMAT][R][NB];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int b = 0; b < NB; b++) acc[m][r][b] = 0.0f;
    // the next item's weights, then this item's products from LDS x
    auto step = [&](const Q8Slice (&now)[NMAT][R], Q8Slice (&next)[NMAT][R], int i, bool load = true) {
        if (load) load_item(next, i + 1);
        const int g = i / nch, c = i - g * nch;
        const int blk = 32 * c + (lane >> 1);
        const bool valid = blk < nb;
        const int k0 = (valid ? blk : 0) * Q8_BLOCK + 16 * (lane & 1);
        float xv[NB][16];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float4* xp = reinterpret_cast<const float4*>(xs + b * n + k0);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 v = xp[q];
                xv[b][4 * q] = valid ? v.x : 0.0f;
                xv[b][4 * q + 1] = valid ? v.y : 0.0f;
                xv[b][4 * q + 2] = valid ? v.z : 0.0f;
                xv[b][4 * q + 3] = valid ? v.w : 0.0f;
            }
        }
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                float wv[16];
#pragma unroll
                for (int q = 0; q < 16; q++) wv[q] = q8_value(now[m][r].q[q >> 2], q & 3);
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    float sum = 0.0f;
#pragma unroll
                    for (int q = 0; q < 16; q++) sum = fmaf(wv[q], xv[b][q], sum);
                    acc[m][r][b] = fmaf(sum, now[m][r].scale, acc[m][r][b]);
                }
            }
        if (c == nch - 1 || i == i1 - 1) {  // the group's last chunk in this run (wave-uniform)
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        float v = acc[m][r][b];
#pragma unroll
                        for (int msk = 32; msk > 0; msk >>= 1) v += __shfl_xor(v, msk);
                        if (lane == 0) red[(((g * R + r) * NMAT + m) * NB + b) * W + wave] = v;
                        acc[m][r][b] = 0.0f;
                    }
        }
    };
    int i = i0;
    if constexpr (EARLY2) {
        // the first item's successor is already in flight
        if (i < i1) step(sa, sb, i, false);
        i++;
        for (; i + 1 < i1; i += 2) {
            step(sb, sa, i);
            step(sa, sb, i + 1);
        }
        if (i < i1) step(sb, sa, i);
    } else {
        for (; i + 1 < i1; i += 2) {
            step(sa, sb, i);
            step(sb, sa, i + 1);
        }
        if (i < i1) step(sa, sb, i);
    }
    if constexpr (NORM) {
        // wave b < NB adds batch row b's partials (loaded in the prologue)
        if (wave < NB) {
            float v = 0.0f;
#pragma unroll
            for (int i = 0; i < PE; i++) v += lane + i * 64 < nm.nparts ? pv[i] : 0.0f;
            for (int p = lane + PE * 64; p < nm.nparts; p += 64) v += nm.ss[(size_t)p * nm.ss_stride + wave];
#pragma unroll
            for (int msk = 32; msk > 0; msk >>= 1) v += __shfl_xor(v, msk);
            if (lane == 0) inv_s[wave] = inv_rms(v, n);
        }
    }
    __syncthreads();

    // epilogue: thread (b, local row il), rows in order within each batch row
    // (16 consecutive lanes per 16-row tile for the residual partials)
    static_assert(!RESID || UG % 16 == 0, "residual partials are per 16 rows");
    for (int t = threadIdx.x; t < NB * rows; t += NT) {
        const int b = t / rows, il = t - b * rows;
        float sum[NMAT], pair[2] = {0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < W; w++) v += red[((il * NMAT + m) * NB + b) * W + w];
            sum[m] = NORM ? v * inv_s[b] : v;
        }
        if constexpr (ROPE) {
            // RoPE pairs are local rows (il, il ^ 1)
#pragma unroll
            for (int m = 0; m < 2; m++) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < W; w++) v += red[(((il ^ 1) * NMAT + m) * NB + b) * W + w];
                pair[m] = NORM ? v * inv_s[b] : v;
            }
        }
        store_row_sums<NMAT, SWIGLU, RESID, ROPE>(grp, resid, rope, b, row0 + il, sum, pair);
    }
}

// Batches of more than 4 rows (full-row products) on the bf16 matrix cores
// at fp32 accuracy.  An int8 weight is exact in bf16, and an fp32 activation
// is the exact sum of three bf16 numbers: hi = its upper 16 bits, mid = the
// upper 16 bits of the remainder and lo = what is left (each step keeps 8
// significant bits; 24 in all).  Each product q * part is exact in the fp32
// accumulator, so three v_mfma_f32_16x16x32_bf16 (lo, mid, hi; 32 k = one
// block each) give the block's sum sum_k q[k] * x[k] with fp32 accumulation,
// which is then scaled: acc += scale * sum (the reference scales each weight
// before the product, src/model_q8.cpp:106-112; the two agree to fp32
// rounding).  Per instruction, A = x parts (lane l: batch row l%16, k =
// 8*(l/16) + i of the block) and B = the block's weights (lane l: weight row
// l%16, bytes 4 + 8*(l/16) .. +8 of its 36), so the accumulator leaves lane l
// holding out[batch 4*(l/16) + j][row l%16] and every lane scales by the
// scale of its own row.
//
// A workgroup owns 16 rows of each group member and 16 or 32 batch rows (BT
// tiles of 16; larger batches add workgroups along y); MMA_WAVES waves take the rows' blocks U at a time,
// round-robin.  A wave's rounds are pipelined: it loads a round's x (an L2
// read) and then issues the next round's weight loads before computing, so
// one round of weights is always in flight behind the one in use (the x
// loads go first because a wait covers every older load).  At the end the
// waves' tiles are added through LDS in a fixed wave order, one thread per
// (member, batch row, row), and the shared epilogue runs.  8 waves: at the
// model shapes the rows' blocks are few (24 for k = 768), and 16 waves spent
// longer in that reduction than they saved in the loop (Llama-2-110M-shaped
// step at batch 32: 0.598 against 0.607 ms; 7B-shaped at batch 8: 4.36
// against 4.41 ms; 4 waves: 0.625 and 4.83 ms).
constexpr int MMA_WAVES = 8;
constexpr int MMA_TILE_STRIDE = 20;  // floats per batch row of a staged tile (stores hit 64 distinct banks)


// Eight int8 weights (two words, k order) as bf16.
__device__ __forceinline__ bf16x8 q8_bf16(uint32_t w0, uint32_t w1) {
    u32x4 r;
    r[0] = bf16_pair(q8_value(w0, 0), q8_value(w0, 1));
    r[1] = bf16_pair(q8_value(w0, 2), q8_value(w0, 3));
    r[2] = bf16_pair(q8_value(w1, 0), q8_value(w1, 1));
    r[3] = bf16_pair(q8_value(w1, 2), q8_value(w1, 3));
    return __builtin_bit_cast(bf16x8, r);
}

// Blocks per wave per round: two rounds of weights and x stay within 128
// registers (two 8-wave workgroups per CU).
template <int NMAT, int BT>
constexpr int mma_unroll() {
    return BT == 1 ? (NMAT == 3 ? 1 : 2) : 1;
}
constexpr int MMA_MAX_BT = 2;       // batch tiles per workgroup (more rows: more workgroups along y)
constexpr int MMA_NORM_MAX_N = 8192;  // rms weights staged in LDS (larger n: the fp32 kernel)

// One round of a wave: weights and x of U blocks.
template <int NMAT, int BT, int U>
struct MmaRound {
    uint32_t q[U][NMAT][2];
    float scale[U][NMAT];
    float x[BT][U][8];
};

template <int NMAT, int BT, bool TILED, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
__global__ __launch_bounds__(64 * MMA_WAVES) void q8_mma_kernel(Q8Group grp, const float* __restrict__ x, int batch,
                                                                int n, Q8Norm nm, Q8Resid resid, Q8Rope rope) {
    constexpr int U = mma_unroll<NMAT, BT>();
    constexpr int STRIDE = MMA_WAVES * U;  // blocks per round of the workgroup
    __shared__ float red[MMA_WAVES][NMAT][16 * MMA_TILE_STRIDE];
    __shared__ float norm_s[NORM ? MMA_WAVES * 64 : 1];
    __shared__ float norm_w[NORM ? MMA_NORM_MAX_N : 1];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int row0 = blockIdx.x * 16;
    const int b0 = blockIdx.y * 16 * BT;
    const int nb = n / Q8_BLOCK;
    // Lanes past the batch read the last batch row and rows past a member's
    // end read its last row (finite values, never stored); blocks past the
    // row read the last block, and compute gives them scale 0.
    // (32-bit offsets from the uniform bases: the launcher keeps each matrix
    // and x under 2^32 bytes).  Block blk of this lane: its 8 weights at
    // qoff + blk * BSTEP, its row's scale at soff + blk * BSTEP.
    constexpr uint32_t BSTEP = TILED ? 576 : Q8_BLOCK_BYTES;
    const uint8_t* wbase[NMAT];
    uint32_t qoff[NMAT], soff[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        if constexpr (TILED) {
            const uint32_t rec = (uint32_t)min((int)blockIdx.x, (grp.d[m] + 15) / 16 - 1) * nb * 576;
            wbase[m] = grp.wt[m];
            qoff[m] = rec + 64 + 8 * lane;
            soff[m] = rec + 4 * r;
        } else {
            const uint32_t row = (uint32_t)min(row0 + r, grp.d[m] - 1) * nb * Q8_BLOCK_BYTES;
            wbase[m] = grp.w[m];
            qoff[m] = row + 4 + 8 * g;
            soff[m] = row;
        }
    }
    uint32_t xrow[BT];
#pragma unroll
    for (int t = 0; t < BT; t++) xrow[t] = (uint32_t)min(b0 + t * 16 + r, batch - 1) * n + 8 * g;
    f32x4 acc[NMAT][BT];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int t = 0; t < BT; t++) acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

    using Round = MmaRound<NMAT, BT, U>;
    auto load_round = [&](Round& R, int base) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool valid = base + u < nb;
            const int blk = valid ? base + u : nb - 1;
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const uint2 q = *reinterpret_cast<const uint2*>(wbase[m] + (qoff[m] + (uint32_t)blk * BSTEP));
                R.q[u][m][0] = q.x;
                R.q[u][m][1] = q.y;
                R.scale[u][m] = *reinterpret_cast<const float*>(wbase[m] + (soff[m] + (uint32_t)blk * BSTEP));
            }
#pragma unroll
            for (int t = 0; t < BT; t++) {
                const float4 a = *reinterpret_cast<const float4*>(x + (xrow[t] + blk * Q8_BLOCK));
                const float4 c = *reinterpret_cast<const float4*>(x + (xrow[t] + blk * Q8_BLOCK + 4));
                R.x[t][u][0] = a.x, R.x[t][u][1] = a.y, R.x[t][u][2] = a.z, R.x[t][u][3] = a.w;
                R.x[t][u][4] = c.x, R.x[t][u][5] = c.y, R.x[t][u][6] = c.z, R.x[t][u][7] = c.w;
            }
        }
    };
    // per block: its weights as bf16, then per batch tile the split x and
    // NMAT independent chains (lo, mid, hi), scaled into the accumulators
    auto compute = [&](const Round& R, int base) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            bf16x8 wb[NMAT];
#pragma unroll
            for (int m = 0; m < NMAT; m++) wb[m] = q8_bf16(R.q[u][m][0], R.q[u][m][1]);
#pragma unroll
            for (int t = 0; t < BT; t++) {
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = R.x[t][u][i];
                if constexpr (NORM) {
                    const float inv = norm_s[t * 16 + r];
                    const int k0 = min(base + u, nb - 1) * Q8_BLOCK + 8 * g;
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] = norm_w[k0 + i] * (inv * v[i]);
                }
                bf16x8 xh, xm, xl;
                split3(v, xh, xm, xl);
                f32x4 sm[NMAT];
#pragma unroll
                for (int m = 0; m < NMAT; m++) sm[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wb[m], zero, 0, 0, 0);
#pragma unroll
                for (int m = 0; m < NMAT; m++) sm[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xm, wb[m], sm[m], 0, 0, 0);
#pragma unroll
                for (int m = 0; m < NMAT; m++) sm[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wb[m], sm[m], 0, 0, 0);
                // a block past the row (a repeat of the last one) counts 0;
                // tested here, not at the load, so nothing waits on the loads
                // of the round in flight
#pragma unroll
                for (int m = 0; m < NMAT; m++) {
                    const float sc = base + u < nb ? R.scale[u][m] : 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[m][t][j] = fmaf(sc, sm[m][j], acc[m][t][j]);
                }
            }
        }
    };
    // The two round buffers alternate: the next round's loads are all issued
    // before the current round is computed.
    Round ra, rb;
    int base = wave * U;
    if (base < nb) load_round(ra, base);  // in flight while the norm prologue runs
    if constexpr (NORM) {
        // thread (row j = tid % 64, class c = tid / 64) adds partials c, c + 16, ...;
        // row j's class sums are then added in class order: norm_s[j] = inv_rms
        // The rms weights' loads and the partials' loads go out together
        // (only wave-uniform branches around them), then the stores.  Lanes
        // past the workgroup's batch rows reread a real row's partials (same
        // addresses as a lane that needs them) and store 0.
        const int j = threadIdx.x & 63, c = threadIdx.x >> 6;
        constexpr int NW = MMA_NORM_MAX_N / (64 * MMA_WAVES);
        const int nw = (n + 64 * MMA_WAVES - 1) / (64 * MMA_WAVES);  // uniform
        float wv[NW];
#pragma unroll
        for (int i = 0; i < NW; i++)
            if (i < nw) wv[i] = nm.weight[min((int)threadIdx.x + i * 64 * MMA_WAVES, n - 1)];
        const int prow = min(b0 + min(j, 16 * BT - 1), batch - 1);
        // 4 loads per class cover up to 64 partials (rows of 1024): fewer wasted loads
        const float ps = nm.nparts <= 4 * MMA_WAVES ? partial_sum_unbranched<4>(nm, prow, c, MMA_WAVES)
                                                    : partial_sum_unbranched<16>(nm, prow, c, MMA_WAVES);
        norm_s[c * 64 + j] = j < 16 * BT && b0 + j < batch ? ps : 0.0f;
#pragma unroll
        for (int i = 0; i < NW; i++)
            if (i < nw) norm_w[threadIdx.x + i * 64 * MMA_WAVES] = wv[i];
        __syncthreads();
        float ss = 0.0f;
#pragma unroll
        for (int cc = 0; cc < MMA_WAVES; cc++) ss += norm_s[cc * 64 + lane];
        __syncthreads();
        if (wave == 0) norm_s[lane] = inv_rms(ss, n);
        __syncthreads();
    }
    while (base < nb) {  // uniform
        if (base + STRIDE < nb) load_round(rb, base + STRIDE);
        compute(ra, base);
        base += STRIDE;
        if (base >= nb) break;
        if (base + STRIDE < nb) load_round(ra, base + STRIDE);
        compute(rb, base);
        base += STRIDE;
    }

    // Per batch tile: every wave stages its tile (lane l: batch rows
    // 4*(l/16)+j, row l%16), then thread (m, b = (tid/16)%16, i = tid%16)
    // adds the waves in order; the epilogue runs on the first 256 threads.
    __shared__ float sums[NMAT][256];
#pragma unroll
    for (int t = 0; t < BT; t++) {
        if (b0 + t * 16 >= batch) break;  // uniform
        if (t > 0) __syncthreads();  // the previous tile's reads are done
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int j = 0; j < 4; j++) red[wave][m][(4 * g + j) * MMA_TILE_STRIDE + r] = acc[m][t][j];
        __syncthreads();
        for (int e = threadIdx.x; e < NMAT * 256; e += 64 * MMA_WAVES) {
            const int m = e >> 8, bl = (e >> 4) & 15, i = e & 15;
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < MMA_WAVES; w++) v += red[w][m][bl * MMA_TILE_STRIDE + i];
            sums[m][e & 255] = v;
        }
        __syncthreads();
        if (threadIdx.x < 256) {
            const int bl = threadIdx.x >> 4, i = threadIdx.x & 15;
            const int b = b0 + t * 16 + bl;
            if (b < batch) {  // uniform over the 16 threads of batch row b
                float sum[NMAT], pair[2] = {0.0f, 0.0f};
#pragma unroll
                for (int m = 0; m < NMAT; m++) sum[m] = sums[m][threadIdx.x];
                if constexpr (ROPE) {
                    pair[0] = sums[0][threadIdx.x ^ 1];
                    pair[1] = sums[1][threadIdx.x ^ 1];
                }
                store_row_sums<NMAT, SWIGLU, RESID, ROPE>(grp, resid, rope, b, row0 + i, sum, pair);
            }
        }
    }
}

bool use_mma() {
    static const bool on = [] {
        const char* e = getenv("NITRO_Q8_MMA");
        return !(e && e[0] == 'f');  // "f32": the fp32 matrix-core kernel (comparison runs)
    }();
    return on;
}

// Row streaming pays off once a row has at least two 1024-k chunks (both k
// halves busy).  Tiles are small (4R rows), so there are enough of them to
// fill the GPU; past ROWDOT_MAX_GROUPS the workgroups loop over tiles.
constexpr int ROWDOT_MIN_N = 2048;
constexpr int ROWDOT_MAX_GROUPS = 1024;

// NITRO_Q8_GEMV (read once): "slab" sends rows of >= 2048 k to the slab
// kernel, "rowdot" to the row-streaming one; by default they take the flat
// kernel when their activations fit its LDS, else the row-streaming one.
int gemv_choice() {
    static const int c = [] {
        const char* e = getenv("NITRO_Q8_GEMV");
        return e && e[0] == 's' ? 0 : e && e[0] == 'r' ? 1 : 2;
    }();
    return c;
}

int device_cus() {
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

// The flat kernel, if its activations and partial sums fit its LDS budget.
template <int NB, int NMAT, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
bool launch_flat(const Q8Group& grp, const float* x, int n, int dmax, const Q8Norm& nm, const Q8Resid& rs,
                 const Q8Rope& rp, hipStream_t stream) {
    if ((long long)NB * n > flat_x_max<RESID>()) return false;
    const auto kern = q8_flat_kernel<NB, NMAT, SWIGLU, NORM, RESID, ROPE>;
    // workgroups resident per CU at the largest LDS the launch may take
    // (once per instantiation; the dynamic LDS limit is raised to that size)
    static const int per_cu = [kern] {
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            flat_lds_max<RESID>());
        int blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kern, 64 * flat_waves<RESID>(), flat_lds_max<RESID>()) !=
            hipSuccess)
            blocks = 1;
        return std::max(blocks, 1);
    }();
    constexpr int UG = flat_unit_rows<RESID>();
    const int units = (dmax + UG - 1) / UG;
    const int groups = std::min(units, per_cu * device_cus());
    const long long rows_max = (long long)(units + groups - 1) / groups * UG;
    const size_t lds = ((size_t)NB * n + (size_t)rows_max * NMAT * NB * flat_waves<RESID>()) * sizeof(float);
    if (lds > (size_t)flat_lds_max<RESID>()) return false;
    hipLaunchKernelGGL(kern, dim3((unsigned)groups), dim3(64 * flat_waves<RESID>()), lds, stream, grp, x, n, dmax, nm, rs,
                       rp);
    return true;
}

template <int NB, int NMAT, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
void launch_gemv(const Q8Group& grp, const float* x, int n, int dmax, const Q8Norm& nm, const Q8Resid& rs,
                 const Q8Rope& rp, hipStream_t stream) {
    if (n >= ROWDOT_MIN_N && gemv_choice() == 2 &&
        launch_flat<NB, NMAT, SWIGLU, NORM, RESID, ROPE>(grp, x, n, dmax, nm, rs, rp, stream))
        return;
    if (n >= ROWDOT_MIN_N && gemv_choice() >= 1) {
        constexpr int ROWS = ROWDOT_SETS * 4 * rowdot_rows<NB, NMAT>();
        const int ntiles = (dmax + ROWS - 1) / ROWS;
        const dim3 grid((unsigned)std::min(ntiles, ROWDOT_MAX_GROUPS)), block(512);
        hipLaunchKernelGGL((q8_rowdot_kernel<NB, NMAT, SWIGLU, NORM, RESID, ROPE>), grid, block, 0, stream, grp, x,
                           n, ntiles, nm, rs, rp);
        return;
    }
    const dim3 grid((unsigned)((dmax + 15) / 16)), block(64 * GEMV_WAVES);
    hipLaunchKernelGGL((q8_gemv_kernel<NB, NMAT, SWIGLU, NORM, RESID, ROPE>), grid, block, 0, stream, grp, x, n, nm,
                       rs, rp);
}

template <int NMAT, bool TILED, bool SWIGLU, bool NORM, bool RESID, bool ROPE>
void launch_mma(const Q8Group& grp, const float* x, int batch, int n, int dmax, const Q8Norm& nm, const Q8Resid& rs,
                const Q8Rope& rp, hipStream_t stream) {
    const dim3 block(64 * MMA_WAVES);
    const unsigned tiles = (unsigned)((dmax + 15) / 16);
    // (three members with two batch tiles would exceed the registers)
    constexpr int BT = NMAT == 3 ? 1 : MMA_MAX_BT;
    // Two batch tiles per workgroup halve its weight loads; one per workgroup
    // doubles the workgroups, which pays while those still fit the GPU: the
    // Llama-2-110M shapes at batch 32 (768-row matrices: 96 workgroups rather
    // than 48) took the model step from 0.703 to 0.610 ms, while a 4096 x 4096
    // product at batch 32 (256 tiles) took 32.6 us against 25.2 with two.
    const unsigned btiles = (unsigned)((batch + 15) / 16);
    if (BT == 1 || btiles == 1 || (long long)tiles * btiles <= device_cus()) {
        hipLaunchKernelGGL((q8_mma_kernel<NMAT, 1, TILED, SWIGLU, NORM, RESID, ROPE>), dim3(tiles, btiles), block,
                           0, stream, grp, x, batch, n, nm, rs, rp);
    } else {
        const dim3 g2(tiles, (unsigned)((batch + 16 * BT - 1) / (16 * BT)));
        hipLaunchKernelGGL((q8_mma_kernel<NMAT, BT, TILED, SWIGLU, NORM, RESID, ROPE>), g2, block, 0, stream, grp, x,
                           batch, n, nm, rs, rp);
    }
}

// The tile layout (Q8Tiled): workgroup (block, tile), lane c copies run c
// (8 weights of row 16*tile + c%16) and lanes 0..15 the scales.
__global__ __launch_bounds__(64) void q8_tile_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ tiled,
                                                     int d, int nb, int tiles) {
    const int blk = blockIdx.x, c = threadIdx.x;
    for (int tile = blockIdx.y; tile < tiles; tile += gridDim.y) {
        const int row = tile * 16 + (c & 15);
        uint32_t q0 = 0, q1 = 0;
        float sc = 0.0f;
        if (row < d) {
            const uint8_t* bp = w + ((size_t)row * nb + blk) * Q8_BLOCK_BYTES;
            const uint32_t* qp = reinterpret_cast<const uint32_t*>(bp + 4 + 8 * (c >> 4));
            q0 = qp[0];
            q1 = qp[1];
            sc = *reinterpret_cast<const float*>(bp);
        }
        uint8_t* rec = tiled + ((size_t)tile * nb + blk) * 576;
        *reinterpret_cast<uint2*>(rec + 64 + 8 * c) = make_uint2(q0, q1);
        if (c < 16) *reinterpret_cast<float*>(rec + 4 * c) = sc;
    }
}

template <int NMAT, bool SWIGLU, bool NORM, bool RESID, bool ROPE = false>
void launch_group(const Q8Group& grp, const float* x, int batch, int n, int dmax, bool last, const Q8Norm& nm,
                  const Q8Resid& rs, hipStream_t stream, const Q8Rope& rp = Q8Rope{}) {
    const dim3 grid((unsigned)((dmax + 15) / 16),
                    (unsigned)((batch + 16 * Q8_MAX_BTILES - 1) / (16 * Q8_MAX_BTILES)));
    const dim3 block(64 * Q8_WAVES);
    if (last) {
        hipLaunchKernelGGL((q8_last_kernel<NMAT, SWIGLU, NORM, RESID, ROPE>), grid, block, 0, stream, grp, x, batch,
                           n, nm, rs, rp);
        return;
    }
    if (batch <= Q8_GEMV_MAX_BATCH) {
        switch (batch) {
            case 1: launch_gemv<1, NMAT, SWIGLU, NORM, RESID, ROPE>(grp, x, n, dmax, nm, rs, rp, stream); break;
            case 2: launch_gemv<2, NMAT, SWIGLU, NORM, RESID, ROPE>(grp, x, n, dmax, nm, rs, rp, stream); break;
            case 3: launch_gemv<3, NMAT, SWIGLU, NORM, RESID, ROPE>(grp, x, n, dmax, nm, rs, rp, stream); break;
            default: launch_gemv<4, NMAT, SWIGLU, NORM, RESID, ROPE>(grp, x, n, dmax, nm, rs, rp, stream); break;
        }
        return;
    }
    // the bf16 kernel addresses weights and x with 32-bit offsets
    const bool mma_fits = q8_tiled_bytes(dmax, n) < (1ull << 32) && (size_t)batch * n < (1ull << 32) &&
                          (!NORM || n <= MMA_NORM_MAX_N);
    if (use_mma() && mma_fits) {
        bool tiled = true;
        for (int m = 0; m < NMAT; m++) tiled = tiled && grp.wt[m] != nullptr;
        if (tiled)
            launch_mma<NMAT, true, SWIGLU, NORM, RESID, ROPE>(grp, x, batch, n, dmax, nm, rs, rp, stream);
        else
            launch_mma<NMAT, false, SWIGLU, NORM, RESID, ROPE>(grp, x, batch, n, dmax, nm, rs, rp, stream);
        return;
    }
    hipLaunchKernelGGL((q8_matmul_kernel<NMAT, SWIGLU, NORM, RESID, ROPE>), grid, block, 0, stream, grp, x, batch, n,
                       nm, rs, rp);
}

}  // namespace

hipError_t launch_q8_tile(const void* w, void* tiled, int d, int n, hipStream_t stream) {
    if (d <= 0 || n <= 0 || n % Q8_BLOCK) return hipErrorInvalidValue;
    const int tiles = (d + 15) / 16;
    hipLaunchKernelGGL(q8_tile_kernel, dim3((unsigned)(n / Q8_BLOCK), (unsigned)std::min(tiles, 65535)), dim3(64), 0,
                       stream, static_cast<const uint8_t*>(w), static_cast<uint8_t*>(tiled), d, n / Q8_BLOCK, tiles);
    return hipGetLastError();
}

hipError_t launch_q8_matmul(const void* w, const float* x, float* out, int batch, int n, int d,
                            bool last_block_only, hipStream_t stream) {
    Q8Group grp{{static_cast<const uint8_t*>(w), nullptr, nullptr}, {out, nullptr, nullptr}, {d, 0, 0}, {}};
    launch_group<1, false, false, false>(grp, x, batch, n, d, last_block_only, Q8Norm{}, Q8Resid{}, stream);
    return hipGetLastError();
}

hipError_t launch_q8_residual(const void* w, const float* in, float* x, float* ss, int batch, int n, int d,
                              bool last_block_only, hipStream_t stream, const void* w_tiled) {
    Q8Group grp{{static_cast<const uint8_t*>(w), nullptr, nullptr},
                {x, nullptr, nullptr},
                {d, 0, 0},
                {static_cast<const uint8_t*>(w_tiled), nullptr, nullptr}};
    launch_group<1, false, false, true>(grp, in, batch, n, d, last_block_only, Q8Norm{}, Q8Resid{ss, batch},
                                        stream);
    return hipGetLastError();
}

hipError_t launch_q8_qkv(const void* const* w, const float* x, float* out_q, const int* d, int batch, int n,
                         bool last_block_only, const Q8Norm& nm, const Q8Rope& rope, hipStream_t stream,
                         const Q8Tiled& tiled) {
    if (!nm.weight || !rope.freq_real || d[1] != d[2] || d[0] % 32 || d[1] % 32) return hipErrorInvalidValue;
    Q8Group grp{};
    for (int m = 0; m < 3; m++) {
        grp.w[m] = static_cast<const uint8_t*>(w[m]);
        grp.d[m] = d[m];
        grp.wt[m] = static_cast<const uint8_t*>(tiled.w[m]);
    }
    grp.out[0] = out_q;  // k and v go to the pools
    const int dmax = std::max(d[0], d[1]);
    launch_group<3, false, true, false, true>(grp, x, batch, n, dmax, last_block_only, nm, Q8Resid{}, stream, rope);
    return hipGetLastError();
}

hipError_t launch_q8_swiglu(const void* w1, const void* w3, const float* x, float* hb, int batch, int n,
                            int hidden, bool last_block_only, const Q8Norm& nm, hipStream_t stream,
                            const Q8Tiled& tiled) {
    Q8Group grp{{static_cast<const uint8_t*>(w1), static_cast<const uint8_t*>(w3), nullptr},
                {hb, nullptr, nullptr},
                {hidden, hidden, 0},
                {static_cast<const uint8_t*>(tiled.w[0]), static_cast<const uint8_t*>(tiled.w[1]), nullptr}};
    if (!nm.weight) return hipErrorInvalidValue;
    launch_group<2, true, true, false>(grp, x, batch, n, hidden, last_block_only, nm, Q8Resid{}, stream);
    return hipGetLastError();
}

}  // namespace nitro
