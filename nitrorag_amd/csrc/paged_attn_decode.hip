// Batched paged-attention decode for gfx950 (MI355X).
//
// Computes, for every (sequence b, query head h), what the reference's
// forward_decode_batch attention computes (src/model_q8.cpp:625-662):
//   s_t = q_h . k_t / sqrt(hd) over keys t = 0..pos_b (pages via the block
//   table, kv head h / (H/Hkv)), p = softmax(s), o_h = sum_t p_t v_t.
//
// Design (bandwidth-bound: K and V are read exactly once per query head):
//  - Grid: one workgroup of W wavefronts per (b, h, split), W = 4..16 chosen
//    per launch (more waves per sequence when the batch is small, so enough
//    loads are in flight and long contexts finish in few rounds).  A split is
//    a run of `tiles_per_split` tiles of TILE consecutive context rows; waves
//    take the split's tiles round-robin.
//  - Lane layout: LG = 8 lanes share one K/V row (16 for hd=256) so that every
//    global_load_dwordx4 reads whole 128-byte lines; a lane holds hd/LG floats
//    of each of its RL rows (columns c*4 + j*4*LG).  The 64/LG row groups of a
//    wave take interleaved rows of a TILE-row tile (64, 32, 16, 8 rows for
//    hd = 32, 64, 128, 256); all 16 K/V float4 loads of a tile are issued
//    before use.
//  - q.k: hd/LG FMAs per lane and row, then a DPP butterfly across the LG lanes.
//  - Softmax: every lane group keeps its own running (max, sum, acc) in base 2
//    (q is pre-scaled by log2(e)/sqrt(hd)); groups, then waves (through LDS),
//    then splits are merged with the usual rescaling.  No score scratch.
//  - Split-K: when one split per (b, h) would leave the GPU underfilled, each
//    workgroup writes (m, l, acc[hd]) for its split and a second, small
//    kernel merges the splits.  With one split the workgroup writes the output
//    directly and decode is a single launch.  (Merging inside the kernel by
//    the last-arriving workgroup needs agent-scope release/acquire fences,
//    which write back and invalidate the whole XCD L2 per workgroup on
//    gfx950; measured, that halved throughput at two splits.)
//  - The split's block-table slice is staged in LDS once; page ids outside
//    the pool are counted in *bad_pages and their rows skipped (no fault).
#include <hip/hip_runtime.h>

#include <cmath>

#include "device_pool.hpp"

namespace nitro {
namespace {

constexpr int MAX_WAVES = 16;
constexpr int MAX_THREADS = 64 * MAX_WAVES;

template <int HD>
struct DecodeGeom {
    // LG lanes share a K/V row so that one load instruction reads whole
    // 128-byte lines (8 lanes x 16 B; 16 lanes for hd=256, two lines).  Each
    // lane holds NF4 float4 of a row (columns c*4 + j*4*LG) for RL rows per
    // tile: RL*NF4 = 8 float4 of K and 8 of V in flight per lane.
    static constexpr int LG = HD <= 128 ? 8 : 16;
    static constexpr int NF4 = HD / (4 * LG);
    static constexpr int RL = 8 / NF4;
    static constexpr int GROUPS = 64 / LG;  // row groups per wave
    static constexpr int TILE = RL * GROUPS;
    static_assert(NF4 >= 1 && RL * NF4 == 8, "head_dim 32, 64, 128 or 256");
};

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over the LG consecutive lanes of a group (result in every lane).
template <int LG>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (LG >= 2) x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (LG >= 4) x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (LG >= 8) x += dpp_mov<0x141>(x);  // row_half_mirror: other quad of the 8
    if constexpr (LG >= 16) x += dpp_mov<0x140>(x); // row_mirror: other 8 of the 16
    return x;
}

__device__ __forceinline__ float dot4(float4 a, float4 b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    acc = fmaf(a.w, b.w, acc);
    return acc;
}

typedef float f4v __attribute__((ext_vector_type(4)));

// K/V row loads.  STREAM issues them non-temporal (global_load_dwordx4 ... nt):
// lines read once per launch are not kept in L2 / MALL, which raises the
// achievable streaming rate; plain loads keep lines that other workgroups read
// again (pages shared between sequences, query heads of one KV group).
template <bool STREAM>
__device__ __forceinline__ float4 load_kv(const float* p) {
    if constexpr (STREAM) {
        const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
        return make_float4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const float4*>(p);
    }
}

__device__ __forceinline__ float scale_of(float m, float m_new) {
    return m == -INFINITY ? 0.0f : exp2f(m - m_new);
}

// QH query heads of one KV head per workgroup (QH = 1 for MHA): each K/V
// row is loaded once and scored against all QH queries.  QH > 1 needs about
// twice the registers, so those workgroups hold at most 8 waves.
template <int HD, int QH, bool STREAM>
__global__ __launch_bounds__(QH == 1 ? MAX_THREADS : MAX_THREADS / 2) void paged_attn_decode_kernel(
    DecodeLaunch a) {
    using G = DecodeGeom<HD>;
    constexpr int LG = G::LG, NF4 = G::NF4, RL = G::RL, GROUPS = G::GROUPS, TILE = G::TILE;
    constexpr int MAXW = QH == 1 ? MAX_WAVES : MAX_WAVES / 2;
    __shared__ int32_t s_pages[DECODE_MAX_SPLIT_PAGES];
    __shared__ float s_acc[MAXW][QH][HD];
    __shared__ float s_m[MAXW][QH], s_l[MAXW][QH];
    const int waves = blockDim.x >> 6;
    const int threads = blockDim.x;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane / LG;
    const int c = lane % LG;

    // Work order: ((b*Hkv + kv_h)*splits + split)*(kv_mul/QH) + r; the
    // workgroup serves query heads h0 .. h0+QH-1, h0 = kv_h*kv_mul + r*QH, so
    // the workgroups that read one K/V range are consecutive.  With
    // xcd_remap, block ids are dealt to the 8 XCDs round-robin, so XCD x takes
    // the x-th contiguous eighth of that order: workgroups sharing a K/V range
    // run together on one XCD and re-read it from its L2.
    int w = blockIdx.x;
    if (a.xcd_remap) {
        const int n = gridDim.x, per = n >> 3, rem = n & 7;
        const int x = w & 7;
        w = x * per + min(x, rem) + (w >> 3);
    }
    const int hsubs = a.kv_mul / QH;
    const int r = w % hsubs;
    const int rest = w / hsubs;
    const int split = rest % a.num_splits;
    const int grp = rest / a.num_splits;  // b*Hkv + kv_h
    const int n_kv = a.n_heads / a.kv_mul;
    const int b = grp / n_kv;
    const int kv_h = grp - b * n_kv;
    const int bh0 = b * a.n_heads + kv_h * a.kv_mul + r * QH;
    // The position, q and this split's block-table slice are independent
    // loads: issue them together.  The slice is read speculatively over the
    // split's whole page range (clipped to the table row) and only the
    // entries below the context length are validated and used.
    constexpr int TBL_PER_THREAD = DECODE_MAX_SPLIT_PAGES / 256;  // >= 4 waves per workgroup
    const int tile_begin = split * a.tiles_per_split;
    const int page_begin = (tile_begin * TILE) >> 4;
    const int spec_end = min(a.max_pages, ((tile_begin + a.tiles_per_split) * TILE + 15) >> 4);
    const int32_t* trow = a.tables + (size_t)b * a.max_pages;
    int tv[TBL_PER_THREAD];
#pragma unroll
    for (int k = 0; k < TBL_PER_THREAD; k++) {
        const int i = threadIdx.x + k * threads;
        tv[k] = i < spec_end - page_begin ? trow[page_begin + i] : -1;
    }
    const int ctx = a.positions[b] + 1;

    // q slices of this lane, pre-scaled to base-2 logits.
    float4 qv[QH][NF4];
#pragma unroll
    for (int qi = 0; qi < QH; qi++) {
        const float* qp = a.q + (size_t)(bh0 + qi) * HD;
#pragma unroll
        for (int j = 0; j < NF4; j++) {
            float4 t = *reinterpret_cast<const float4*>(qp + (c + j * LG) * 4);
            qv[qi][j] = make_float4(t.x * a.qscale, t.y * a.qscale, t.z * a.qscale, t.w * a.qscale);
        }
    }

    const int n_tiles = (ctx + TILE - 1) / TILE;
    if (tile_begin >= n_tiles) return;  // uniform for the workgroup
    const int tile_end = min(n_tiles, tile_begin + a.tiles_per_split);
    const int splits_b = (n_tiles + a.tiles_per_split - 1) / a.tiles_per_split;

    // Used part of the slice -> LDS (page ids checked against the pool size).
    const int page_end = ((min(ctx, tile_end * TILE) - 1) >> 4) + 1;
#pragma unroll
    for (int k = 0; k < TBL_PER_THREAD; k++) {
        const int i = threadIdx.x + k * threads;
        if (i < page_end - page_begin) {
            int p = tv[k];
            if ((unsigned)p >= (unsigned)a.num_pages) {
                atomicAdd(a.bad_pages, 1);
                p = -1;
            }
            s_pages[i] = p;
        }
    }
    __syncthreads();

    const float* kbase = a.k_pool + a.layer_off + (size_t)kv_h * HD;
    const float* vbase = a.v_pool + a.layer_off + (size_t)kv_h * HD;

    float m[QH], l[QH];
    float4 acc[QH][NF4];
#pragma unroll
    for (int qi = 0; qi < QH; qi++) {
        m[qi] = -INFINITY;
        l[qi] = 0.0f;
#pragma unroll
        for (int j = 0; j < NF4; j++) acc[qi][j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    for (int t = tile_begin + wave; t < tile_end; t += waves) {
        float4 kr[RL][NF4], vr[RL][NF4];
        bool valid[RL];
        bool any = false;
#pragma unroll
        for (int i = 0; i < RL; i++) {
            const int row = t * TILE + g + i * GROUPS;
            int page = row < ctx ? s_pages[(row >> 4) - page_begin] : -1;
            valid[i] = page >= 0;
            any |= valid[i];
            if (valid[i]) {
                const size_t off = (size_t)page * a.page_stride + (size_t)(row & 15) * a.kv_dim;
#pragma unroll
                for (int j = 0; j < NF4; j++) {
                    kr[i][j] = load_kv<STREAM>(kbase + off + (c + j * LG) * 4);
                    vr[i][j] = load_kv<STREAM>(vbase + off + (c + j * LG) * 4);
                }
            } else {
#pragma unroll
                for (int j = 0; j < NF4; j++) {
                    kr[i][j] = make_float4(0.f, 0.f, 0.f, 0.f);
                    vr[i][j] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        }
        // Rows are valid or not for the whole lane group (same rows), so this
        // skip is uniform across the lanes that the DPP sums combine.
        if (!any) continue;
#pragma unroll
        for (int qi = 0; qi < QH; qi++) {
            float s[RL];
#pragma unroll
            for (int i = 0; i < RL; i++) {
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < NF4; j++) d = dot4(qv[qi][j], kr[i][j], d);
                d = group_sum<LG>(d);
                s[i] = valid[i] ? d : -INFINITY;
            }
            float m_new = m[qi];
#pragma unroll
            for (int i = 0; i < RL; i++) m_new = fmaxf(m_new, s[i]);
            const float alpha = scale_of(m[qi], m_new);
            float p[RL];
            float psum = 0.0f;
#pragma unroll
            for (int i = 0; i < RL; i++) {
                p[i] = valid[i] ? exp2f(s[i] - m_new) : 0.0f;
                psum += p[i];
            }
            l[qi] = l[qi] * alpha + psum;
#pragma unroll
            for (int j = 0; j < NF4; j++) {
                float4 o = make_float4(acc[qi][j].x * alpha, acc[qi][j].y * alpha,
                                       acc[qi][j].z * alpha, acc[qi][j].w * alpha);
#pragma unroll
                for (int i = 0; i < RL; i++) {
                    o.x = fmaf(p[i], vr[i][j].x, o.x);
                    o.y = fmaf(p[i], vr[i][j].y, o.y);
                    o.z = fmaf(p[i], vr[i][j].z, o.z);
                    o.w = fmaf(p[i], vr[i][j].w, o.w);
                }
                acc[qi][j] = o;
            }
            m[qi] = m_new;
        }
    }

    // Merge the lane groups of the wave (lanes with equal c, across g).
#pragma unroll
    for (int qi = 0; qi < QH; qi++) {
#pragma unroll
        for (int mask = LG; mask < 64; mask <<= 1) {
            const float mo = __shfl_xor(m[qi], mask);
            const float lo = __shfl_xor(l[qi], mask);
            const float mm = fmaxf(m[qi], mo);
            const float f = scale_of(m[qi], mm), fo = scale_of(mo, mm);
            l[qi] = l[qi] * f + lo * fo;
#pragma unroll
            for (int j = 0; j < NF4; j++) {
                float4 o;
                o.x = __shfl_xor(acc[qi][j].x, mask);
                o.y = __shfl_xor(acc[qi][j].y, mask);
                o.z = __shfl_xor(acc[qi][j].z, mask);
                o.w = __shfl_xor(acc[qi][j].w, mask);
                acc[qi][j] = make_float4(acc[qi][j].x * f + o.x * fo, acc[qi][j].y * f + o.y * fo,
                                         acc[qi][j].z * f + o.z * fo, acc[qi][j].w * f + o.w * fo);
            }
            m[qi] = mm;
        }
        if (g == 0) {
#pragma unroll
            for (int j = 0; j < NF4; j++)
                *reinterpret_cast<float4*>(&s_acc[wave][qi][(c + j * LG) * 4]) = acc[qi][j];
            if (c == 0) {
                s_m[wave][qi] = m[qi];
                s_l[wave][qi] = l[qi];
            }
        }
    }
    __syncthreads();

    // Merge the waves: thread o owns output column o % HD of head o / HD.
    for (int o = threadIdx.x; o < QH * HD; o += threads) {
        const int qi = o / HD, d = o - qi * HD;
        float M = -INFINITY, L = 0.0f, A = 0.0f;
        for (int wv = 0; wv < waves; wv++) M = fmaxf(M, s_m[wv][qi]);
        for (int wv = 0; wv < waves; wv++) {
            const float f = scale_of(s_m[wv][qi], M);
            L += s_l[wv][qi] * f;
            A += s_acc[wv][qi][d] * f;
        }
        const int bh = bh0 + qi;
        if (splits_b == 1) {
            a.out[(size_t)bh * HD + d] = A / L;
        } else {
            float* part = a.partials + ((size_t)bh * a.num_splits + split) * (HD + 2);
            part[d] = A;
            if (d == 0) {
                part[HD] = M;
                part[HD + 1] = L;
            }
        }
    }
}

// Merges the per-split partials of every (b, h) that has more than one split.
template <int HD>
__global__ __launch_bounds__(HD < 64 ? 64 : HD) void paged_attn_decode_merge_kernel(DecodeLaunch a) {
    constexpr int TILE = DecodeGeom<HD>::TILE;
    const int bh = blockIdx.x;
    const int b = bh / a.n_heads;
    const int ctx = a.positions[b] + 1;
    const int n_tiles = (ctx + TILE - 1) / TILE;
    const int splits_b = (n_tiles + a.tiles_per_split - 1) / a.tiles_per_split;
    const int d = threadIdx.x;
    if (splits_b <= 1 || d >= HD) return;  // single split: written by the main kernel
    const float* pb = a.partials + (size_t)bh * a.num_splits * (HD + 2);
    float M = -INFINITY;
    for (int sp = 0; sp < splits_b; sp++) M = fmaxf(M, pb[sp * (HD + 2) + HD]);
    float L = 0.0f, A = 0.0f;
    for (int sp = 0; sp < splits_b; sp++) {
        const float* ps = pb + sp * (HD + 2);
        const float f = scale_of(ps[HD], M);
        L += ps[HD + 1] * f;
        A += ps[d] * f;
    }
    a.out[(size_t)bh * HD + d] = A / L;
}

}  // namespace

int decode_max_heads_per_wg(int head_dim) {
    return head_dim <= 64 ? 8 : head_dim == 128 ? 4 : 2;  // QH * head_dim <= 512
}

int decode_tile_rows(int head_dim) {
    switch (head_dim) {
        case 32: return DecodeGeom<32>::TILE;
        case 64: return DecodeGeom<64>::TILE;
        case 128: return DecodeGeom<128>::TILE;
        case 256: return DecodeGeom<256>::TILE;
        default: return 0;
    }
}

template <int HD, int QH>
static void launch_main(const DecodeLaunch& a, dim3 grid, hipStream_t stream) {
    if (a.stream_kv)
        hipLaunchKernelGGL((paged_attn_decode_kernel<HD, QH, true>), grid, dim3(64 * a.waves), 0,
                           stream, a);
    else
        hipLaunchKernelGGL((paged_attn_decode_kernel<HD, QH, false>), grid, dim3(64 * a.waves), 0,
                           stream, a);
}

template <int HD>
static hipError_t launch_hd(const DecodeLaunch& a, hipStream_t stream) {
    if (a.heads_per_wg < 1 || a.kv_mul % a.heads_per_wg != 0 ||
        a.heads_per_wg > decode_max_heads_per_wg(HD) ||
        (a.heads_per_wg > 1 && a.waves > MAX_WAVES / 2))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((size_t)a.batch * (a.n_heads / a.heads_per_wg) * a.num_splits));
    switch (a.heads_per_wg) {
        case 1: launch_main<HD, 1>(a, grid, stream); break;
        case 2: launch_main<HD, 2>(a, grid, stream); break;
        case 4:
            if constexpr (4 * HD <= 512) launch_main<HD, 4>(a, grid, stream);
            break;
        case 8:
            if constexpr (8 * HD <= 512) launch_main<HD, 8>(a, grid, stream);
            break;
        default: return hipErrorInvalidValue;
    }
    if (a.num_splits > 1) {
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(paged_attn_decode_merge_kernel<HD>, dim3((unsigned)(a.batch * a.n_heads)),
                           dim3(HD < 64 ? 64 : HD), 0, stream, a);
    }
    return hipGetLastError();
}

hipError_t launch_paged_attn_decode(const DecodeLaunch& a, hipStream_t stream) {
    // >= 4 waves: the block-table slice (<= DECODE_MAX_SPLIT_PAGES entries) is
    // loaded at most 4 entries per thread.
    if (a.waves < 4 || a.waves > MAX_WAVES || 64 * a.waves < a.head_dim) return hipErrorInvalidValue;
    switch (a.head_dim) {
        case 32: return launch_hd<32>(a, stream);
        case 64: return launch_hd<64>(a, stream);
        case 128: return launch_hd<128>(a, stream);
        case 256: return launch_hd<256>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace nitro
