// Causal paged-attention prefill for gfx950 (MI355X).
//
// Computes what the reference's forward_prefill_chunk attention computes
// (src/model_q8.cpp:485-523) for a batch of chunks: the token at position
// pos = start_pos + t attends keys 0..pos of its sequence (prefix-hit pages,
// earlier chunks and the chunk's own rows, already scattered into the pool).
//
// Three kernels, all at fp32 accuracy:
//  - paged_attn_prefill_x3_kernel (hd 32/64/128, the default): the bf16
//    matrix cores on exact three-part bf16 splits of Q, K, V and P (its
//    comment below);
//  - paged_attn_prefill_mfma_kernel (NITRO_PREFILL_KERNEL=mfma32): the fp32
//    matrix cores;
//  - paged_attn_prefill_kernel (hd 256, or NITRO_PREFILL_KERNEL=valu): fp32
//    VALU FMAs.
//
// paged_attn_prefill_mfma_kernel<hd, QT, KSPLIT, BNM> runs both matrix
// products on v_mfma_f32_16x16x4_f32 (fp32 inputs, fp32 accumulate):
//  - Work item = 64 query rows of one chunk x one head; a workgroup has QT = 4
//    query sub-tiles of 16 rows x KSPLIT = 2 key groups (8 waves; two
//    workgroups per CU interleave their phases).  Keys stream in tiles of BNM
//    rows (64 for hd <= 64, 32 for hd 128) staged in LDS with a row stride of
//    hd+4 floats (conflict-free reads below), the next tile prefetched into
//    registers while the current one is consumed.  The workgroup's
//    block-table slice is staged in LDS once.
//  - Per 16-key block a wave computes S^T = K Q^T (16 keys x 16 queries):
//    lane l supplies K[key l%16][d] and Q[query l%16][d] for d = g*hd/4 + kk
//    (g = l/16; the reduction order over d is permuted so each lane's K reads
//    are contiguous ds_read_b128).  The accumulator leaves lane l holding
//    S[query l%16][keys 4g..4g+3], so a query's statistics live in the four
//    lanes l%16 (reduced with gfx950's permlane16/32 swaps, no LDS), and the
//    same four registers are exactly the B operand of O^T += V^T P^T (keys
//    4g+kk at step kk), whose output leaves lane l holding
//    O[query l%16][16n+4g..+3]: rescaling by the query's factor is lane-local.
//  - A wave's blocks of a tile are scored together (independent S chains,
//    one softmax step).  Online softmax in base 2 (q pre-scaled by
//    log2(e)/sqrt(hd)); blocks wholly below the diagonal skip the causal mask,
//    and the running max is moved (rescaling O and l) only when it grows by
//    more than 8 (log2 units).  Blocks above a wave's last query are skipped
//    wave-uniformly: no per-lane skip may surround an MFMA.
//  - Key groups hand (m, l, O) to key group 0 through LDS at the end.
//
// paged_attn_prefill_kernel<HDP, FULL> (any head size that is a multiple of
// 4 up to 256; used for hd 256 and sizes other than 32/64/128) is the VALU form:
//  - A work item is up to BM=64 query rows of one chunk; grid = (work items,
//    heads).  The host sorts work items by key count, longest first.
//  - 256 threads: 4 lanes per query row, each lane holding hd/4 of q and of
//    the output accumulator (float4 slots c, c+4, ... so the 4 lanes of a row
//    read 64 contiguous bytes of an LDS row: no bank conflicts).
//  - Keys stream in tiles of BN=32 rows (two pages) staged in LDS through the
//    block table; the next tile is prefetched into registers while the current
//    one is consumed.
//  - Scores in base 2 (q pre-scaled by log2(e)/sqrt(hd)), causal mask per row,
//    online softmax rescaled once per 8 keys.
#include <hip/hip_runtime.h>

#include <type_traits>

#include <cmath>

#include "bf16_split.hpp"
#include "device_pool.hpp"

namespace nitro {
namespace {

constexpr int BM = 64;
constexpr int BN = 32;
constexpr int THREADS = 256;  // BM rows x 4 lanes
constexpr int KCHUNK = 8;

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float sum4(float x) {
    x += dpp_mov<0xB1>(x);  // lane ^ 1
    x += dpp_mov<0x4E>(x);  // lane ^ 2
    return x;
}

__device__ __forceinline__ float scale_of(float m, float m_new) {
    return m == -INFINITY ? 0.0f : exp2f(m - m_new);
}

// HDP: the head size rounded up to 32, 64, 128 or 256 (the LDS and register
// layout); FULL: the head size is HDP, otherwise columns past it are loaded
// as zero and never stored.
template <int HDP, bool FULL>
__global__ __launch_bounds__(THREADS) void paged_attn_prefill_kernel(PrefillLaunch a) {
    constexpr int HD = HDP;
    constexpr int F4 = HD / 4;               // float4 per row
    constexpr int SLOTS = F4 / 4;            // float4 per lane
    constexpr int LOADS = BN * F4 / THREADS; // float4 per thread per tile per matrix
    static_assert(LOADS >= 1 && BN * F4 % THREADS == 0, "tile shape");
    __shared__ float4 ks[BN][F4];
    __shared__ float4 vs[BN][F4];
    const int hd = FULL ? HD : a.head_dim;
    const int hd4 = hd / 4;

    // 1-D grid, heads fastest: the work list is sorted longest first, so every
    // head of the longest items is dispatched before any shorter item.
    const int item = blockIdx.x / a.n_heads;
    const int h = blockIdx.x - item * a.n_heads;
    const int seq = a.work[2 * item];
    const int q0 = a.work[2 * item + 1];
    const int kv_h = h / a.kv_mul;
    const int start = a.start_pos[seq];
    const int qcount = min(BM, a.num_tokens[seq] - q0);
    const int row = threadIdx.x >> 2;
    const int c = threadIdx.x & 3;
    const int last_pos = start + q0 + qcount - 1;
    const int my_pos = start + q0 + min(row, qcount - 1);
    const int32_t* trow = a.tables + (size_t)seq * a.max_pages;
    const int n_tiles = last_pos / BN + 1;
    const size_t dim = (size_t)a.n_heads * hd;
    const size_t qrow = (size_t)(a.row_off[seq] + q0 + min(row, qcount - 1));

    float4 qv[SLOTS];
    {
        const float4* qp = reinterpret_cast<const float4*>(a.q + qrow * dim + (size_t)h * hd);
#pragma unroll
        for (int e = 0; e < SLOTS; e++) {
            float4 t = FULL || c + 4 * e < hd4 ? qp[c + 4 * e] : make_float4(0.f, 0.f, 0.f, 0.f);
            qv[e] = make_float4(t.x * a.qscale, t.y * a.qscale, t.z * a.qscale, t.w * a.qscale);
        }
    }
    float4 acc[SLOTS];
#pragma unroll
    for (int e = 0; e < SLOTS; e++) acc[e] = make_float4(0.f, 0.f, 0.f, 0.f);
    float m = -INFINITY, l = 0.0f;

    const float* kbase = a.k_pool + a.layer_off + (size_t)kv_h * hd;
    const float* vbase = a.v_pool + a.layer_off + (size_t)kv_h * hd;
    float4 kreg[LOADS], vreg[LOADS];

    // Fetch: the tile's page ids first, then every K/V load unconditionally
    // (a key past the context or on a bad page reads page 0 instead), so no
    // load waits behind another; kmask records which rows are real and the
    // LDS store zeroes the rest.  At hd 256 (256 VGPRs) each row is looked up
    // and loaded in turn, under the page check, and fetch zeroes the rest
    // itself: the other form measured 5-10% slower there.
    static_assert(LOADS <= 32, "validity mask");
    uint32_t kmask = 0;
    auto fetch = [&](int tile) {
        kmask = 0;
        if constexpr (HD == 256) {
#pragma unroll
            for (int i = 0; i < LOADS; i++) {
                const int f = threadIdx.x + i * THREADS;
                const int r = f / F4, col = f % F4;
                const int key = tile * BN + r;
                kreg[i] = vreg[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (key <= last_pos) {
                    const int page = trow[key >> 4];
                    if ((unsigned)page < (unsigned)a.num_pages) {
                        const size_t off = (size_t)page * a.page_stride + (size_t)(key & 15) * a.kv_dim;
                        if (FULL || col < hd4) {
                            kreg[i] = reinterpret_cast<const float4*>(kbase + off)[col];
                            vreg[i] = reinterpret_cast<const float4*>(vbase + off)[col];
                        }
                    } else if (col == 0) {
                        atomicAdd(a.bad_pages, 1);
                    }
                }
            }
        } else {
            int page[LOADS];
#pragma unroll
            for (int i = 0; i < LOADS; i++)
                page[i] = trow[min(tile * BN + (int)(threadIdx.x + i * THREADS) / F4, last_pos) >> 4];
#pragma unroll
            for (int i = 0; i < LOADS; i++) {
                const int f = threadIdx.x + i * THREADS;
                const int r = f / F4, col = f % F4;
                const int key = tile * BN + r;
                const bool in = key <= last_pos;
                const bool ok = in && (unsigned)page[i] < (unsigned)a.num_pages;
                if (in && !ok && col == 0) atomicAdd(a.bad_pages, 1);
                const bool colok = FULL || col < hd4;  // a column past the head reads column 0
                kmask |= (uint32_t)(ok && colok) << i;
                const size_t off = ok ? (size_t)page[i] * a.page_stride + (size_t)(key & 15) * a.kv_dim : 0;
                kreg[i] = reinterpret_cast<const float4*>(kbase + off)[colok ? col : 0];
                vreg[i] = reinterpret_cast<const float4*>(vbase + off)[colok ? col : 0];
            }
        }
    };

    fetch(0);
    for (int tile = 0; tile < n_tiles; tile++) {
        __syncthreads();  // previous tile fully consumed
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int f = threadIdx.x + i * THREADS;
            const bool ok = HD == 256 || ((kmask >> i) & 1);  // hd 256: fetch zeroed the rest
            ks[f / F4][f % F4] = ok ? kreg[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            vs[f / F4][f % F4] = ok ? vreg[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
        if (tile + 1 < n_tiles) fetch(tile + 1);

        const int key0 = tile * BN;
#pragma unroll 1
        for (int jc = 0; jc < BN; jc += KCHUNK) {
            if (key0 + jc > my_pos) break;  // row-uniform (the 4 lanes of a row agree)
            float s[KCHUNK];
            float cmax = -INFINITY;
#pragma unroll
            for (int jj = 0; jj < KCHUNK; jj++) {
                const int j = jc + jj;
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < SLOTS; e++) {
                    const float4 kk = ks[j][c + 4 * e];
                    d = fmaf(qv[e].x, kk.x, d);
                    d = fmaf(qv[e].y, kk.y, d);
                    d = fmaf(qv[e].z, kk.z, d);
                    d = fmaf(qv[e].w, kk.w, d);
                }
                d = sum4(d);
                s[jj] = (key0 + j <= my_pos) ? d : -INFINITY;
                cmax = fmaxf(cmax, s[jj]);
            }
            const float m_new = fmaxf(m, cmax);
            const float alpha = scale_of(m, m_new);
            l *= alpha;
#pragma unroll
            for (int e = 0; e < SLOTS; e++)
                acc[e] = make_float4(acc[e].x * alpha, acc[e].y * alpha, acc[e].z * alpha,
                                     acc[e].w * alpha);
#pragma unroll
            for (int jj = 0; jj < KCHUNK; jj++) {
                const float p = s[jj] == -INFINITY ? 0.0f : exp2f(s[jj] - m_new);
                l += p;
#pragma unroll
                for (int e = 0; e < SLOTS; e++) {
                    const float4 vv = vs[jc + jj][c + 4 * e];
                    acc[e].x = fmaf(p, vv.x, acc[e].x);
                    acc[e].y = fmaf(p, vv.y, acc[e].y);
                    acc[e].z = fmaf(p, vv.z, acc[e].z);
                    acc[e].w = fmaf(p, vv.w, acc[e].w);
                }
            }
            m = m_new;
        }
    }

    if (row < qcount) {
        const float inv = 1.0f / l;
        float4* op = reinterpret_cast<float4*>(a.out + qrow * dim + (size_t)h * hd);
#pragma unroll
        for (int e = 0; e < SLOTS; e++)
            if (FULL || c + 4 * e < hd4)
                op[c + 4 * e] = make_float4(acc[e].x * inv, acc[e].y * inv, acc[e].z * inv, acc[e].w * inv);
    }
}


typedef float f32x4 __attribute__((ext_vector_type(4)));

// The larger of a and b, NaN if either is (v_maximum3_f32).  fmaxf ignores a
// NaN operand, so in IEEE mode the compiler first quiets each operand that is
// not the result of arithmetic (an MFMA or permute result) with an extra
// v_max_f32 x, x.  A NaN score makes the softmax NaN either way.
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Max / sum over the four lanes l%16 + 16g (g = 0..3) of a wave, on gfx950's
// row-swap permutes (VALU only; no LDS round trip).  permlane16_swap(x, x)
// returns rows (0,0,2,2) and (1,1,3,3); permlane32_swap(y, y) returns halves
// (lo,lo) and (hi,hi).
__device__ __forceinline__ float max_over_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = max_nan(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return max_nan(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float sum_over_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}


// The MFMA kernel's lazy rescaling threshold (log2 units): the running max
// used as the exponent reference moves only when a block's max exceeds it by
// more than this, so unnormalised weights stay <= 2^8.
constexpr float kLazyRescaleLog2 = 8.0f;

// Block-table entries a prefill workgroup keeps in LDS (32k tokens); pages
// beyond that are read from the table in global memory.
constexpr int TABLE_LDS = 2048;
// An MFMA-kernel workgroup is QT query sub-tiles of 16 rows x KSPLIT key
// groups of waves, each key group taking every KSPLIT-th 16-key block of a
// BNM-key tile.  A 64-query work item is served by 4/QT workgroups.
template <int HD, int QT, int KSPLIT, int BNM>
__global__ __launch_bounds__(64 * QT * KSPLIT) void paged_attn_prefill_mfma_kernel(PrefillLaunch a) {
    constexpr int QSPLIT = 4 / QT;             // workgroups per 64-query work item
    constexpr int NT = 64 * QT * KSPLIT;
    constexpr int KB = BNM / 16;               // 16-key blocks per tile
    constexpr int F4 = HD / 4;                 // float4 per K/V row
    constexpr int DG = HD / 4;                 // d values per lane group (S^T reduction steps)
    constexpr int NB = HD / 16;                // 16-column blocks of the output
    constexpr int STRIDE = HD + 4;             // padded LDS row (floats)
    constexpr int LOADS = BNM * F4 / NT;       // float4 per thread per tile per matrix
    static_assert(LOADS >= 1 && BNM * F4 % NT == 0, "tile shape");
    static_assert(KB % KSPLIT == 0, "key blocks split evenly over key groups");
    constexpr int NBW = KB / KSPLIT;           // 16-key blocks per wave per tile
    // K and V tiles in one array; after the key loop the same LDS holds the
    // partials (16 queries x HD per sub-tile) of key groups 1..KSPLIT-1.
    static_assert(QT * QSPLIT == 4 && NT <= 1024, "workgroup shape");
    static_assert((KSPLIT - 1) * QT * 16 * HD <= 2 * BNM * STRIDE, "partials fit the tile LDS");
    __shared__ __attribute__((aligned(16))) float kv_lds[2 * BNM * STRIDE];
    float* const ks = kv_lds;
    float* const vs = kv_lds + BNM * STRIDE;
    __shared__ int32_t s_table[TABLE_LDS];
    __shared__ float s_ml[KSPLIT > 1 ? QT * (KSPLIT - 1) * 16 * 2 : 1];

    // blockIdx.x = (item * QSPLIT + part) * n_heads + h.  Part 0 takes the
    // item's highest query sub-tiles (its longest key range), so dispatch
    // stays longest first.
    const int h = blockIdx.x % a.n_heads;
    const int ip = blockIdx.x / a.n_heads;
    const int item = ip / QSPLIT;
    const int sub0 = (QSPLIT - 1 - ip % QSPLIT) * QT;  // first query sub-tile of this workgroup
    const int seq = a.work[2 * item];
    const int q0 = a.work[2 * item + 1];
    const int kv_h = h / a.kv_mul;
    const int start = a.start_pos[seq];
    const int qcount = min(BM, a.num_tokens[seq] - q0);  // queries of the work item
    if (sub0 * 16 >= qcount) return;  // no query in this part (uniform)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int qs = wave % QT;    // query sub-tile of this workgroup (16 rows)
    const int kg = wave / QT;    // key group: blocks kg, kg + KSPLIT, ... of each tile
    const int ql = lane & 15;    // query within the sub-tile
    const int g = lane >> 4;     // lane group: K/V rows 4g..4g+3 of a block, d slice g
    const int row = (sub0 + qs) * 16 + ql;  // query row within the work item
    const int last_pos = start + q0 + min((sub0 + QT) * 16, qcount) - 1;
    const int my_pos = start + q0 + min(row, qcount - 1);
    const int wave_last = start + q0 + min((sub0 + qs) * 16 + 15, qcount - 1);
    const int wave_first = start + q0 + min((sub0 + qs) * 16, qcount - 1);
    const int32_t* trow = a.tables + (size_t)seq * a.max_pages;
    const int n_tiles = last_pos / BNM + 1;
    const size_t dim = (size_t)a.n_heads * HD;
    const size_t qrow = (size_t)(a.row_off[seq] + q0 + min(row, qcount - 1));

    // The workgroup's block-table slice -> LDS (read once instead of per tile).
    const int n_pages = min((last_pos >> 4) + 1, TABLE_LDS);
    for (int i = threadIdx.x; i < n_pages; i += NT) s_table[i] = trow[i];
    __syncthreads();

    float qv[DG];
    {
        const float4* qp = reinterpret_cast<const float4*>(a.q + qrow * dim + (size_t)h * HD + g * DG);
#pragma unroll
        for (int i = 0; i < DG / 4; i++) {
            const float4 t = qp[i];
            qv[4 * i + 0] = t.x * a.qscale;
            qv[4 * i + 1] = t.y * a.qscale;
            qv[4 * i + 2] = t.z * a.qscale;
            qv[4 * i + 3] = t.w * a.qscale;
        }
    }
    f32x4 acc[NB];
#pragma unroll
    for (int n = 0; n < NB; n++) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.0f;

    const float* kbase = a.k_pool + a.layer_off + (size_t)kv_h * HD;
    const float* vbase = a.v_pool + a.layer_off + (size_t)kv_h * HD;
    float4 kreg[LOADS], vreg[LOADS];

    // Fetch: a tile's page ids are all looked up first, then every K/V load
    // is issued unconditionally (a key past the context or on a bad page reads
    // page 0 instead), so no load waits behind another; kmask records which
    // rows are real and the LDS store zeroes the rest.  The ids come from the
    // LDS copy of the table when all of the work item's pages are in it
    // (block-uniform); otherwise pages past the copy are read from memory.
    static_assert(LOADS <= 32, "validity mask");
    const bool table_in_lds = (last_pos >> 4) < TABLE_LDS;
    uint32_t kmask = 0;
    auto fetch_with = [&](int tile, auto page_of) {
        int page[LOADS];
#pragma unroll
        for (int i = 0; i < LOADS; i++)
            page[i] = page_of(min(tile * BNM + (int)(threadIdx.x + i * NT) / F4, last_pos));
        kmask = 0;
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int f = threadIdx.x + i * NT;
            const int r = f / F4, col = f % F4;
            const int key = tile * BNM + r;
            const bool in = key <= last_pos;
            const bool ok = in && (unsigned)page[i] < (unsigned)a.num_pages;
            if (in && !ok && col == 0) atomicAdd(a.bad_pages, 1);
            kmask |= (uint32_t)ok << i;
            const size_t off = ok ? (size_t)page[i] * a.page_stride + (size_t)(key & 15) * a.kv_dim : 0;
            kreg[i] = reinterpret_cast<const float4*>(kbase + off)[col];
            vreg[i] = reinterpret_cast<const float4*>(vbase + off)[col];
        }
    };
    auto fetch = [&](int tile) {
        if (table_in_lds)
            fetch_with(tile, [&](int key) { return s_table[key >> 4]; });
        else
            fetch_with(tile, [&](int key) {
                const int pi = key >> 4;
                return pi < TABLE_LDS ? s_table[pi] : trow[pi];
            });
    };

    fetch(0);
    for (int tile = 0; tile < n_tiles; tile++) {
        __syncthreads();  // previous tile fully consumed
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int f = threadIdx.x + i * NT;
            const int r = f / F4, col = f % F4;
            const bool ok = (kmask >> i) & 1;
            *reinterpret_cast<float4*>(&ks[r * STRIDE + col * 4]) = ok ? kreg[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            *reinterpret_cast<float4*>(&vs[r * STRIDE + col * 4]) = ok ? vreg[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
        if (tile + 1 < n_tiles) fetch(tile + 1);

        // This wave's blocks of the tile, kg + j*KSPLIT (j < NBW), are scored
        // together: NBW independent S chains, then one softmax step over
        // their 4*NBW scores per lane, then the PV products.  Blocks are in
        // increasing key order, so the ones some query of the wave can see
        // (first key <= wave_last) are a prefix of nvb blocks.
        int nvb = 0;
#pragma unroll
        for (int j = 0; j < NBW; j++)
            if (tile * BNM + (kg + j * KSPLIT) * 16 <= wave_last) nvb = j + 1;
        if (nvb > 0) {  // wave-uniform
            f32x4 st[NBW];
#pragma unroll
            for (int j = 0; j < NBW; j++) {
                // S^T block: lane holds S[query ql][keys key0_j + 4g + r], r = 0..3
                st[j] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (j < nvb) {  // wave-uniform
                    const float* krow = &ks[((kg + j * KSPLIT) * 16 + ql) * STRIDE + g * DG];
#pragma unroll
                    for (int i = 0; i < DG / 4; i++) {
                        const float4 kk4 = *reinterpret_cast<const float4*>(krow + 4 * i);
                        st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk4.x, qv[4 * i + 0], st[j], 0, 0, 0);
                        st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk4.y, qv[4 * i + 1], st[j], 0, 0, 0);
                        st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk4.z, qv[4 * i + 2], st[j], 0, 0, 0);
                        st[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk4.w, qv[4 * i + 3], st[j], 0, 0, 0);
                    }
                }
            }
            const int last_key0 = tile * BNM + (kg + (nvb - 1) * KSPLIT) * 16;
            float p[NBW][4];
            if (nvb == NBW && last_key0 + 15 <= wave_first) {
                // Every key of the blocks precedes every query of the wave: no
                // mask, finite scores.  The reference point m moves (rescaling
                // O and l) only when some row's max exceeds it by more than
                // kLazyRescaleLog2; otherwise p = 2^(s - m) <= 2^8 and O, l
                // carry the same common factor, which the final O/l cancels.
                float bmax = fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3]));
#pragma unroll
                for (int j = 1; j < NBW; j++)
                    bmax = fmaxf(bmax, fmaxf(fmaxf(st[j][0], st[j][1]), fmaxf(st[j][2], st[j][3])));
                bmax = max_over_rows(bmax);
                if (__builtin_amdgcn_ballot_w64(bmax > m + kLazyRescaleLog2) != 0) {  // wave-uniform
                    const float m_new = fmaxf(m, bmax);
                    const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // m = -inf: 0
                    lsum *= alpha;
#pragma unroll
                    for (int n = 0; n < NB; n++) acc[n] *= alpha;
                    m = m_new;
                }
#pragma unroll
                for (int j = 0; j < NBW; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) p[j][r] = __builtin_amdgcn_exp2f(st[j][r] - m);
            } else {
                // Diagonal blocks: causal mask per element (and blocks past the
                // wave's last query contribute nothing).  m_new stays -inf for a
                // query none of whose keys so far precede it (possible in key
                // groups > 0); alpha and p are then 0.  No lane may skip the
                // MFMAs: their operands are shared across lanes.
                float sm[NBW][4];
                float bmax = -INFINITY;
#pragma unroll
                for (int j = 0; j < NBW; j++) {
                    const int kj = tile * BNM + (kg + j * KSPLIT) * 16 + 4 * g;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        sm[j][r] = (j < nvb && kj + r <= my_pos) ? st[j][r] : -INFINITY;
                        bmax = fmaxf(bmax, sm[j][r]);
                    }
                }
                bmax = max_over_rows(bmax);
                const float m_new = fmaxf(m, bmax);
                const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - m_new);
#pragma unroll
                for (int j = 0; j < NBW; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        p[j][r] = sm[j][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sm[j][r] - m_new);
                lsum *= alpha;
#pragma unroll
                for (int n = 0; n < NB; n++) acc[n] *= alpha;
                m = m_new;
            }
#pragma unroll
            for (int j = 0; j < NBW; j++) lsum += (p[j][0] + p[j][1]) + (p[j][2] + p[j][3]);
#pragma unroll
            for (int j = 0; j < NBW; j++) {
                if (j < nvb) {  // wave-uniform
                    const int kb = kg + j * KSPLIT;
#pragma unroll
                    for (int n = 0; n < NB; n++) {
                        f32x4 o = acc[n];
                        const float* vcol = &vs[(kb * 16 + 4 * g) * STRIDE + 16 * n + ql];
#pragma unroll
                        for (int kk = 0; kk < 4; kk++)
                            o = __builtin_amdgcn_mfma_f32_16x16x4f32(vcol[kk * STRIDE], p[j][kk], o, 0, 0, 0);
                        acc[n] = o;
                    }
                }
            }
        }
    }

    lsum = sum_over_rows(lsum);
    if constexpr (KSPLIT > 1) {
        // Key groups 1.. hand (m, l, O) to key group 0 through LDS (the K tile area).
        __syncthreads();  // every wave is done with the K/V tiles
        float* part = kv_lds;  // [(KSPLIT-1) x QT sub-tiles][16 queries][HD]
        if (kg > 0) {
            const int slot = (kg - 1) * QT + qs;
            float* o = part + (size_t)slot * 16 * HD + ql * HD;
#pragma unroll
            for (int n = 0; n < NB; n++)
                *reinterpret_cast<float4*>(o + 16 * n + 4 * g) =
                    make_float4(acc[n][0], acc[n][1], acc[n][2], acc[n][3]);
            if (g == 0) {
                s_ml[(slot * 16 + ql) * 2 + 0] = m;
                s_ml[(slot * 16 + ql) * 2 + 1] = lsum;
            }
        }
        __syncthreads();
        if (kg > 0) return;
#pragma unroll
        for (int k = 1; k < KSPLIT; k++) {
            const int slot = (k - 1) * QT + qs;
            const float mo = s_ml[(slot * 16 + ql) * 2 + 0];
            const float lo = s_ml[(slot * 16 + ql) * 2 + 1];
            const float mm = fmaxf(m, mo);
            const float f = scale_of(m, mm), fo = scale_of(mo, mm);
            lsum = lsum * f + lo * fo;
            const float* o = part + (size_t)slot * 16 * HD + ql * HD;
#pragma unroll
            for (int n = 0; n < NB; n++) {
                const float4 t = *reinterpret_cast<const float4*>(o + 16 * n + 4 * g);
                acc[n] = acc[n] * f + f32x4{t.x, t.y, t.z, t.w} * fo;
            }
            m = mm;
        }
    }
    if (row < qcount) {
        const float inv = 1.0f / lsum;
        float* op = a.out + qrow * dim + (size_t)h * HD;
#pragma unroll
        for (int n = 0; n < NB; n++)
            *reinterpret_cast<float4*>(op + 16 * n + 4 * g) =
                make_float4(acc[n][0] * inv, acc[n][1] * inv, acc[n][2] * inv, acc[n][3] * inv);
    }
}

// paged_attn_prefill_x3_kernel<hd, KSPLIT, BNM>: the MFMA kernel's work
// split and softmax with both products on the bf16 matrix cores at fp32
// accuracy.  Q and K are each split into three bf16 parts (hi, mid, lo;
// exact, 24 significant bits in all), and S = K Q^T takes the six part
// products whose order is at most 2 (hi.hi, hi.mid, mid.hi, hi.lo, mid.mid,
// lo.hi; the dropped ones are below 2^-24 of the total): an error in S moves
// every weight exponentially, so S keeps fp32 accuracy.  V and the
// probabilities P are split into two (hi, mid: 16 significant bits, the rest
// below 2^-16 of each value), and O takes the four products V.P (mid.mid,
// mid.hi, hi.mid, hi.hi): O is a weighted average of V, so relative errors
// of at most 2^-16 in V and P move it by at most about 3e-5 of the values'
// size.  All accumulate in fp32 by v_mfma_f32_16x16x32_bf16, smallest first:
//  - S^T = K Q^T per 16-key block and 32 d: lane l supplies K[key l%16] and
//    Q[query l%16] at d = 32c + 8*(l/16) .. +8, so the accumulator leaves lane
//    l holding S[query l%16][keys 4g..4g+3] (g = l/16) as before;
//  - O^T += V^T P^T per pair of 16-key blocks (32 keys): lane l's B operand
//    is its own probabilities of the two blocks (keys 4g..4g+3 of each), and
//    its A operand V^T[d = 16n + l%16] at the same 8 keys, read from a
//    transposed V tile.
// A workgroup serves one work item of 16*QT query rows (QT = 8: 128 rows,
// the wide work list, so each staged tile serves twice the queries) with QT
// query sub-tiles x KSPLIT key groups of waves.
// K and V are split once, when a tile is staged: three bf16 planes of K and
// two of V in LDS, K as [key][d] and V as [d][key].  K is loaded a float4 of one key row
// per thread; V one d of four consecutive keys per thread (a wave's lanes
// cover consecutive d of a row, so the loads coalesce), which becomes one
// 8-byte store per plane into the transposed tile.
// APPEND (1, 2): the launch also appends the chunk.  The chunk's keys are
// read from the new rows k_new / v_new (the same values, so the output is the
// same as after a separate scatter), and the workgroup of the first head of
// each kv group stores its query rows' K/V into the pool from the registers
// the tile loads left them in.  No workgroup reads those pool rows: the host
// takes this form only when no table entry but the row's own names a page a
// chunk row lands on.  APPEND 1: a batch of fresh prompts (every chunk starts
// at position 0), every key new.  APPEND 2: chunks after cached keys; a key
// below its chunk's start is read from the pool, the others from the new
// rows, chosen per key (a tile may hold both).
template <int HD, int QT, int KSPLIT, int BNM, int APPEND>
// Up to hd 64 two workgroups share a CU (LDS), which takes at most 128
// VGPRs (4 waves per SIMD); hd 128 runs one workgroup per CU.
__global__ __launch_bounds__(64 * QT * KSPLIT, HD <= 64 ? 4 : 1) void paged_attn_prefill_x3_kernel(PrefillLaunch a) {
    constexpr int NT = 64 * QT * KSPLIT;
    constexpr int KB = BNM / 16;               // 16-key blocks per tile
    constexpr int NBW = KB / KSPLIT;           // 16-key blocks per wave per tile
    static_assert(KB % KSPLIT == 0 && NBW % 2 == 0, "a wave's blocks pair up into 32-key products");
    constexpr int F4 = HD / 4;                 // float4 per K/V row
    constexpr int NC = HD / 32;                // 32-d chunks of S
    constexpr int NB = HD / 16;                // 16-column blocks of the output
    // K plane row (bf16; 16-byte aligned rows).  HD + 16 measured 64% fewer
    // LDS bank-conflict cycles than HD + 8 (1.24 M vs 3.41 M per launch on 8
    // prompts of 128-1024 tokens at 12 x 64), equal time there and 1.9% less
    // on a 16384-token prompt at 32 x 128; V^T row pitches of BNM + 4 .. + 36
    // left the count unchanged or raised it.
    constexpr int KST = HD + 16;
    constexpr int VST = BNM + 4;               // V^T plane row (bf16; 8-byte aligned rows, stores spread over banks)
    constexpr int LOADS = BNM * F4 / NT;       // K float4 per thread per tile
    constexpr int VSLOTS = BNM * HD / (4 * NT);  // V (d, 4-key group) slots per thread per tile
    static_assert(LOADS >= 1 && BNM * F4 % NT == 0 && VSLOTS >= 1 && BNM * HD % (4 * NT) == 0, "tile shape");
    constexpr int KPLANE = BNM * KST, VPLANE = HD * VST;
    static_assert((KSPLIT - 1) * QT * 16 * HD * 4 <= (3 * KPLANE + 2 * VPLANE) * 2, "partials fit the tile planes");
    // K in three bf16 planes, V^T in two
    __shared__ __attribute__((aligned(16))) uint16_t kv_lds[3 * KPLANE + 2 * VPLANE];
    uint16_t* const k_lds = kv_lds;
    uint16_t* const v_lds = kv_lds + 3 * KPLANE;
    __shared__ int32_t s_table[TABLE_LDS];
    __shared__ float s_ml[KSPLIT > 1 ? QT * (KSPLIT - 1) * 16 * 2 : 1];
    __shared__ int32_t s_wave_bad[NT / 64];

    const int h = blockIdx.x % a.n_heads;
    const int item = blockIdx.x / a.n_heads;
    const int seq = a.work[2 * item];
    const int q0 = a.work[2 * item + 1];
    const int kv_h = h / a.kv_mul;
    const int start = a.start_pos[seq];
    const int qcount = min(16 * QT, a.num_tokens[seq] - q0);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int qs = wave % QT;
    const int kg = wave / QT;
    const int ql = lane & 15;
    const int g = lane >> 4;
    const int row = qs * 16 + ql;
    const int last_pos = start + q0 + qcount - 1;
    const int my_pos = start + q0 + min(row, qcount - 1);
    const int wave_last = start + q0 + min(qs * 16 + 15, qcount - 1);
    const int wave_first = start + q0 + min(qs * 16, qcount - 1);
    const int32_t* trow = a.tables + (size_t)seq * a.max_pages;
    const int n_tiles = last_pos / BNM + 1;
    const size_t dim = (size_t)a.n_heads * HD;
    const size_t qrow = (size_t)(a.row_off[seq] + q0 + min(row, qcount - 1));

    // This lane's query at d = 32c + 8g .. +8, loaded before the table so the
    // two loads' latencies overlap; it is scaled and split into parts once
    // the first tile's K/V loads are in flight.
    float4 qraw[NC][2];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const float4* src = reinterpret_cast<const float4*>(a.q + qrow * dim + (size_t)h * HD + 32 * c + 8 * g);
        qraw[c][0] = src[0];
        qraw[c][1] = src[1];
    }

    f32x4 acc[NB];
#pragma unroll
    for (int n = 0; n < NB; n++) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.0f;

    const float* kbase = a.k_pool + a.layer_off + (size_t)kv_h * HD;
    const float* vbase = a.v_pool + a.layer_off + (size_t)kv_h * HD;
    float4 kreg[LOADS];
    float vreg[VSLOTS][4];
    // Fetch: a tile's page ids are all looked up first, then every K/V load
    // is issued unconditionally (a key past the context or on a bad page reads
    // page 0 instead), so no load waits behind another; kmask/vmask record
    // which values are real and staging zeroes the rest.  The ids come from
    // the LDS copy of the table when all of the work item's pages are in it
    // (block-uniform); otherwise pages past the copy are read from memory.
    static_assert(LOADS <= 32 && 4 * VSLOTS <= 32, "validity masks");
    constexpr uint32_t KFULL = LOADS == 32 ? ~0u : (1u << LOADS) - 1;
    constexpr uint32_t VFULL = 4 * VSLOTS == 32 ? ~0u : (1u << (4 * VSLOTS)) - 1;
    const bool table_in_lds = (last_pos >> 4) < TABLE_LDS;
    uint32_t kmask = 0, vmask = 0;
    auto fetch_with = [&](int tile, auto page_of) {
        int kpage[LOADS], vpage[VSLOTS];
#pragma unroll
        for (int i = 0; i < LOADS; i++)
            kpage[i] = page_of(min(tile * BNM + (int)(threadIdx.x + i * NT) / F4, last_pos));
#pragma unroll
        for (int i = 0; i < VSLOTS; i++)
            vpage[i] = page_of(min(tile * BNM + 4 * ((int)(threadIdx.x + i * NT) / HD), last_pos));
        kmask = vmask = 0;
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int f = threadIdx.x + i * NT;
            const int r = f / F4, col = f % F4;
            const int key = tile * BNM + r;
            const bool in = key <= last_pos;
            const bool ok = in && (unsigned)kpage[i] < (unsigned)a.num_pages;
            if (in && !ok && col == 0) atomicAdd(a.bad_pages, 1);  // once per key (V reads the same page)
            kmask |= (uint32_t)ok << i;
            const size_t off = ok ? (size_t)kpage[i] * a.page_stride + (size_t)(key & 15) * a.kv_dim : 0;
            kreg[i] = reinterpret_cast<const float4*>(kbase + off)[col];
        }
#pragma unroll
        for (int i = 0; i < VSLOTS; i++) {
            const int sl = threadIdx.x + i * NT;
            const int d = sl % HD, key0 = tile * BNM + 4 * (sl / HD);  // 4 keys, one page
            const bool ok = key0 <= last_pos && (unsigned)vpage[i] < (unsigned)a.num_pages;
            const float* vp = vbase + (ok ? (size_t)vpage[i] * a.page_stride : 0) + (size_t)(key0 & 15) * a.kv_dim + d;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                vreg[i][e] = vp[(size_t)e * a.kv_dim];
                vmask |= (uint32_t)(ok && key0 + e <= last_pos) << (4 * i + e);
            }
        }
    };
    // With the whole table in LDS, a thread's loads differ from tile to tile
    // only in their page ids: its K loads read row (tid / F4) % 16 of a page at
    // column tid % F4, its V slots rows 4 * (tid / HD) % 16 .. +3 at column
    // tid % HD (the strides NT / F4 and 4 * NT / HD are whole pages of keys).
    // Each address is then one 32 x 32 -> 64-bit multiply-add on a base fixed
    // for the launch, where the page stride in bytes fits 32 bits (a page of
    // 16 rows over every layer is far below 4 GiB in practice; otherwise
    // fetch_with runs).
    static_assert((NT / F4) % 16 == 0 && (4 * NT / HD) % 16 == 0 && BNM % 16 == 0,
                  "a thread's rows within a page are the same in every tile");
    const uint32_t stride_b = (uint32_t)((uint64_t)a.page_stride * sizeof(float));
    const char* const kb = reinterpret_cast<const char*>(
        kbase + (size_t)((threadIdx.x / F4) % 16) * a.kv_dim + (threadIdx.x % F4) * 4);
    const char* const vb = reinterpret_cast<const char*>(
        vbase + (size_t)((4 * (threadIdx.x / HD)) % 16) * a.kv_dim + threadIdx.x % HD);
    const size_t vrow_b = (size_t)a.kv_dim * sizeof(float);
    // FULL: every key of the tile is at most last_pos (wave-uniform), so
    // only the page ids decide validity and no index needs clamping.
    // SRC: the keys are read from the pool (POOL) or, in an APPEND launch,
    // from the new rows (NEW), where the sequence's row j holds position
    // start + j, or per key from either (MIXED: below start from the pool).
    // NEW reads by position alone, without the table: its masks record only
    // which keys are real, and staging clears the keys on pages outside the
    // pool (the workgroup knows whether it has any) as the other forms do.
    // A key at page index p and the thread's fixed row is new row 16 p + row
    // - start, i.e. at kb + dk + p * 16 rows: the same per-thread pointer plus
    // a workgroup-uniform offset, so the new rows cost no registers of their
    // own, and MIXED picks one of two offsets from the same pointer.  (An
    // earlier form that read cached keys through a separate pool pointer went
    // past 128 VGPRs into spills.)
    constexpr int POOL = 0, NEW = 1, MIXED = 2;
    const bool appends = APPEND && h % a.kv_mul == 0;
    const int own_first = start + q0;
    const size_t rows16_b = 16 * vrow_b;
    const size_t dk = APPEND ? (size_t)(reinterpret_cast<uintptr_t>(a.k_new + (size_t)a.row_off[seq] * a.kv_dim) -
                                        reinterpret_cast<uintptr_t>(a.k_pool + a.layer_off)) -
                                   (size_t)start * vrow_b
                             : 0;
    const size_t dv = APPEND ? (size_t)(reinterpret_cast<uintptr_t>(a.v_new + (size_t)a.row_off[seq] * a.kv_dim) -
                                        reinterpret_cast<uintptr_t>(a.v_pool + a.layer_off)) -
                                   (size_t)start * vrow_b
                             : 0;
    // NEW over a full tile: a thread's load i of tile t reads page index
    // t * BNM/16 + (its page within the tile) + i * (pages per NT threads),
    // so the address is one per-thread base (kn, vn) plus a block-uniform
    // multiple of the 16-row pitch (scalar arithmetic).
    const char* const kn = kb + dk + (size_t)(uint32_t)((threadIdx.x / F4) >> 4) * rows16_b;
    const char* const vn = vb + dv + (size_t)(uint32_t)((4 * (threadIdx.x / HD)) >> 4) * rows16_b;
    auto fetch_lds_as = [&](int tile, auto full, auto src) __attribute__((always_inline)) {
        constexpr bool FULL = decltype(full)::value;
        constexpr int SRC = decltype(src)::value;
        if constexpr (SRC == NEW && FULL) {
            kmask = KFULL;
            vmask = VFULL;
            // (readfirstlane keeps each page index opaque: folded into kn / vn,
            // the compiler holds a 64-bit base per load and spills them)
#pragma unroll
            for (int i = 0; i < LOADS; i++) {
                const int pg = __builtin_amdgcn_readfirstlane(tile * (BNM / 16) + i * (NT / F4 / 16));
                kreg[i] = *reinterpret_cast<const float4*>(kn + (size_t)(uint32_t)pg * rows16_b);
            }
#pragma unroll
            for (int i = 0; i < VSLOTS; i++) {
                const int pg = __builtin_amdgcn_readfirstlane(tile * (BNM / 16) + i * (4 * NT / HD / 16));
                const char* p = vn + (size_t)(uint32_t)pg * rows16_b;
#pragma unroll
                for (int e = 0; e < 4; e++) vreg[i][e] = *reinterpret_cast<const float*>(p + e * vrow_b);
            }
            return;
        }
        kmask = vmask = 0;
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int key = tile * BNM + (int)(threadIdx.x + i * NT) / F4;
            const int kc = FULL ? key : min(key, last_pos);
            const int page = SRC == NEW ? 0 : s_table[kc >> 4];  // -1: outside the pool
            const bool ok = (FULL || key <= last_pos) && page >= 0;
            kmask |= (uint32_t)ok << i;
            const size_t pool_off = (size_t)(uint32_t)(ok ? page : 0) * stride_b;
            const size_t new_off = dk + (size_t)(uint32_t)(kc >> 4) * rows16_b;
            const size_t off = SRC == POOL                  ? pool_off
                               : SRC == MIXED && kc < start ? pool_off
                                                            : (ok ? new_off : 0);
            kreg[i] = *reinterpret_cast<const float4*>(kb + off);
        }
#pragma unroll
        for (int i = 0; i < VSLOTS; i++) {
            const int key0 = tile * BNM + 4 * ((int)(threadIdx.x + i * NT) / HD);  // 4 keys, one page
            const int kc = FULL ? key0 : min(key0, last_pos);
            const int page = SRC == NEW ? 0 : s_table[kc >> 4];
            const bool ok = (FULL || key0 <= last_pos) && page >= 0;
            const char* vp = vb + (size_t)(uint32_t)(ok ? page : 0) * stride_b;
            const char* vn = vb + (ok ? dv + (size_t)(uint32_t)(kc >> 4) * rows16_b : 0);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // a new row past last_pos is not read (the sequence's rows end there)
                const int ec = FULL ? e : max(0, min(e, last_pos - key0));
                const char* p = SRC == POOL || (SRC == MIXED && key0 + e < start) ? vp + e * vrow_b : vn + ec * vrow_b;
                vreg[i][e] = *reinterpret_cast<const float*>(p);
            }
            if (FULL) {
                vmask |= (ok ? 0xFu : 0u) << (4 * i);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) vmask |= (uint32_t)(ok && key0 + e <= last_pos) << (4 * i + e);
            }
        }
    };
    auto fetch_lds = [&](int tile, auto src) __attribute__((always_inline)) {
        if (tile * BNM + BNM - 1 <= last_pos)
            fetch_lds_as(tile, std::true_type{}, src);
        else
            fetch_lds_as(tile, std::false_type{}, src);
    };
    // APPEND launches are taken only where this holds (host).
    const bool fast_fetch = table_in_lds && (uint64_t)a.page_stride * sizeof(float) < (1ull << 32);
    // inlined: as a call (several forms, two call sites) it measured 4x slower
    auto fetch = [&](int tile) __attribute__((always_inline)) {
        if constexpr (APPEND == 2) {
            fetch_lds(tile, std::integral_constant<int, MIXED>{});
        } else if constexpr (APPEND == 1) {
            fetch_lds(tile, std::integral_constant<int, NEW>{});
        } else if (fast_fetch) {
            fetch_lds(tile, std::integral_constant<int, POOL>{});
        } else {
            fetch_with(tile, [&](int key) {
                const int pi = key >> 4;
                return pi < TABLE_LDS ? s_table[pi] : trow[pi];
            });
        }
    };
    auto mfma = [](const bf16x8& x, const bf16x8& y, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, c, 0, 0, 0);
    };

    // The first tile of the new rows is requested before the table, so the
    // two latencies overlap.  The LDS copy of the table holds -1 for an id
    // outside the pool (counted here, once per workgroup), so the tile fetch
    // checks only the sign.
    if constexpr (APPEND == 1) fetch(0);
    const int n_pages = min((last_pos >> 4) + 1, TABLE_LDS);
    bool bad = false;
    for (int i = threadIdx.x; i < n_pages; i += NT) {
        int p = trow[i];
        if ((unsigned)p >= (unsigned)a.num_pages) {
            atomicAdd(a.bad_pages, 1);
            p = -1;
            bad = true;
        }
        s_table[i] = p;
    }
    // Whether any page of the item is outside the pool: one flag per wave,
    // each written by its own wave, read by all after the barrier.
    const bool wave_bad = __builtin_amdgcn_ballot_w64(bad) != 0;
    if (lane == 0) s_wave_bad[wave] = wave_bad;
    __syncthreads();
    bool any_bad = false;  // block-uniform
#pragma unroll
    for (int w = 0; w < NT / 64; w++) any_bad |= s_wave_bad[w] != 0;
    if constexpr (APPEND != 1) fetch(0);
    bf16x8 qp[3][NC];  // Q (pre-scaled) in parts
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const float4 u = qraw[c][0], w = qraw[c][1];
        const float v[8] = {u.x * a.qscale, u.y * a.qscale, u.z * a.qscale, u.w * a.qscale,
                            w.x * a.qscale, w.y * a.qscale, w.z * a.qscale, w.w * a.qscale};
        split3(v, qp[0][c], qp[1][c], qp[2][c]);
    }
    for (int tile = 0; tile < n_tiles; tile++) {
        __syncthreads();  // previous tile fully consumed
        // Staging and the next tile's loads at a raised wave priority: of the
        // waves sharing a SIMD (two workgroups), the ones staging a tile issue
        // before the ones computing, so the tile's barrier is reached and the
        // next loads go out sooner (8 prompts of 128-1024 tokens at 12 x 64:
        // 50.3 vs 51.6-52.5 us by trace; priority 3, or priority 1 also around
        // the matrix-core blocks, were no better).
        __builtin_amdgcn_s_setprio(1);
        // four values as two bf16 planes (hi, mid), one 8-byte store each
        auto stage4v = [](uint16_t* dst, int plane, const float (&v)[4]) {
            const float r0 = v[0] - upper16(v[0]), r1 = v[1] - upper16(v[1]);
            const float r2 = v[2] - upper16(v[2]), r3 = v[3] - upper16(v[3]);
            *reinterpret_cast<uint2*>(dst) = make_uint2(bf16_pair(v[0], v[1]), bf16_pair(v[2], v[3]));
            *reinterpret_cast<uint2*>(dst + plane) = make_uint2(bf16_pair(r0, r1), bf16_pair(r2, r3));
        };
        // four values as three bf16 planes, one 8-byte store each
        auto stage4 = [](uint16_t* dst, int plane, const float (&v)[4]) {
            const float r0 = v[0] - upper16(v[0]), r1 = v[1] - upper16(v[1]);
            const float r2 = v[2] - upper16(v[2]), r3 = v[3] - upper16(v[3]);
            const float l0 = r0 - upper16(r0), l1 = r1 - upper16(r1);
            const float l2 = r2 - upper16(r2), l3 = r3 - upper16(r3);
            *reinterpret_cast<uint2*>(dst) = make_uint2(bf16_pair(v[0], v[1]), bf16_pair(v[2], v[3]));
            *reinterpret_cast<uint2*>(dst + plane) = make_uint2(bf16_pair(r0, r1), bf16_pair(r2, r3));
            *reinterpret_cast<uint2*>(dst + 2 * plane) = make_uint2(bf16_pair(l0, l1), bf16_pair(l2, l3));
        };
        // the masks are applied only where a wave holds a row to zero
        // (the last tile of a sequence, bad pages): other tiles skip the selects
        auto stage_tile = [&](bool masked) {
#pragma unroll
            for (int i = 0; i < LOADS; i++) {
                const int f = threadIdx.x + i * NT;
                const int r = f / F4, col = f % F4;
                const bool ok = !masked || ((kmask >> i) & 1);
                const float kv4[4] = {ok ? kreg[i].x : 0.f, ok ? kreg[i].y : 0.f, ok ? kreg[i].z : 0.f,
                                      ok ? kreg[i].w : 0.f};
                stage4(&k_lds[r * KST + col * 4], KPLANE, kv4);
            }
#pragma unroll
            for (int i = 0; i < VSLOTS; i++) {
                const int sl = threadIdx.x + i * NT;
                float v4[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v4[e] = !masked || ((vmask >> (4 * i + e)) & 1) ? vreg[i][e] : 0.f;
                stage4v(&v_lds[(sl % HD) * VST + 4 * (sl / HD)], VPLANE, v4);
            }
        };
        if constexpr (APPEND == 1) {
            if (any_bad) {  // block-uniform: keys on pages outside the pool are staged as zero
#pragma unroll
                for (int i = 0; i < LOADS; i++) {
                    const int key = tile * BNM + (int)(threadIdx.x + i * NT) / F4;
                    if (s_table[min(key, last_pos) >> 4] < 0) kmask &= ~(1u << i);
                }
#pragma unroll
                for (int i = 0; i < VSLOTS; i++) {
                    const int key0 = tile * BNM + 4 * ((int)(threadIdx.x + i * NT) / HD);  // 4 keys, one page
                    if (s_table[min(key0, last_pos) >> 4] < 0) vmask &= ~(0xFu << (4 * i));
                }
            }
        }
        if (__builtin_amdgcn_ballot_w64(kmask != KFULL || vmask != VFULL) != 0)  // wave-uniform
            stage_tile(true);
        else
            stage_tile(false);
        if constexpr (APPEND) {
            // The append, by the workgroup of the first head of each kv group:
            // the tile's keys that are this item's query rows (positions
            // own_first .. last_pos) are stored from the registers they were
            // just loaded into, at the pool address the pool form reads them
            // from, as streaming stores (nothing in the launch reads them; 0.6
            // us of 57 on 8 prompts of 128-1024 tokens at 12 x 64).  A row on a
            // page outside the pool is counted once (kv head 0, its first
            // column) and skipped, as the scatter does.
            if (appends && tile * BNM + BNM > own_first) {  // block-uniform
                char* const kw = const_cast<char*>(kb);
                char* const vw = const_cast<char*>(vb);
#pragma unroll
                for (int i = 0; i < LOADS; i++) {
                    const int f = threadIdx.x + i * NT;
                    const int key = tile * BNM + f / F4;
                    if (key >= own_first && key <= last_pos) {
                        const int page = s_table[key >> 4];
                        if (page >= 0)
                            __builtin_nontemporal_store(f32x4{kreg[i].x, kreg[i].y, kreg[i].z, kreg[i].w},
                                                        reinterpret_cast<f32x4*>(kw + (size_t)(uint32_t)page * stride_b));
                        else if (kv_h == 0 && f % F4 == 0)
                            atomicAdd(a.bad_pages, 1);
                    }
                }
#pragma unroll
                for (int i = 0; i < VSLOTS; i++) {
                    const int key0 = tile * BNM + 4 * ((int)(threadIdx.x + i * NT) / HD);  // 4 keys, one page
                    const int page = s_table[min(key0, last_pos) >> 4];
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (key0 + e >= own_first && key0 + e <= last_pos && page >= 0)
                            __builtin_nontemporal_store(
                                vreg[i][e], reinterpret_cast<float*>(vw + (size_t)(uint32_t)page * stride_b + e * vrow_b));
                }
            }
        }
        __syncthreads();
        if (tile + 1 < n_tiles) fetch(tile + 1);
        __builtin_amdgcn_s_setprio(0);

        int nvb = 0;
#pragma unroll
        for (int j = 0; j < NBW; j++)
            if (tile * BNM + (kg + j * KSPLIT) * 16 <= wave_last) nvb = j + 1;
        if (nvb > 0) {  // wave-uniform
            f32x4 st[NBW];
#pragma unroll
            for (int j = 0; j < NBW; j++) {
                st[j] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (j < nvb) {  // wave-uniform
                    const uint16_t* kr = &k_lds[((kg + j * KSPLIT) * 16 + ql) * KST + 8 * g];
#pragma unroll
                    for (int c = 0; c < NC; c++) {
                        const bf16x8 kh = *reinterpret_cast<const bf16x8*>(kr + 32 * c);
                        const bf16x8 km = *reinterpret_cast<const bf16x8*>(kr + KPLANE + 32 * c);
                        const bf16x8 kl = *reinterpret_cast<const bf16x8*>(kr + 2 * KPLANE + 32 * c);
                        st[j] = mfma(kl, qp[0][c], st[j]);
                        st[j] = mfma(km, qp[1][c], st[j]);
                        st[j] = mfma(kh, qp[2][c], st[j]);
                        st[j] = mfma(km, qp[0][c], st[j]);
                        st[j] = mfma(kh, qp[1][c], st[j]);
                        st[j] = mfma(kh, qp[0][c], st[j]);
                    }
                }
            }
            const int last_key0 = tile * BNM + (kg + (nvb - 1) * KSPLIT) * 16;
            float p[NBW][4];
            if (nvb == NBW && last_key0 + 15 <= wave_first) {
                float bmax = max_nan(max_nan(st[0][0], st[0][1]), max_nan(st[0][2], st[0][3]));
#pragma unroll
                for (int j = 1; j < NBW; j++)
                    bmax = max_nan(bmax, max_nan(max_nan(st[j][0], st[j][1]), max_nan(st[j][2], st[j][3])));
                bmax = max_over_rows(bmax);
                if (__builtin_amdgcn_ballot_w64(bmax > m + kLazyRescaleLog2) != 0) {  // wave-uniform
                    const float m_new = max_nan(m, bmax);
                    const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // m = -inf: 0
                    lsum *= alpha;
#pragma unroll
                    for (int n = 0; n < NB; n++) acc[n] *= alpha;
                    m = m_new;
                }
#pragma unroll
                for (int j = 0; j < NBW; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) p[j][r] = __builtin_amdgcn_exp2f(st[j][r] - m);
            } else {
                float sm[NBW][4];
                float bmax = -INFINITY;
#pragma unroll
                for (int j = 0; j < NBW; j++) {
                    const int kj = tile * BNM + (kg + j * KSPLIT) * 16 + 4 * g;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        sm[j][r] = (j < nvb && kj + r <= my_pos) ? st[j][r] : -INFINITY;
                        bmax = max_nan(bmax, sm[j][r]);
                    }
                }
                bmax = max_over_rows(bmax);
                const float m_new = max_nan(m, bmax);
                const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - m_new);
#pragma unroll
                for (int j = 0; j < NBW; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        p[j][r] = sm[j][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sm[j][r] - m_new);
                lsum *= alpha;
#pragma unroll
                for (int n = 0; n < NB; n++) acc[n] *= alpha;
                m = m_new;
            }
#pragma unroll
            for (int j = 0; j < NBW; j++) lsum += (p[j][0] + p[j][1]) + (p[j][2] + p[j][3]);
            // O^T += V^T P^T over block pairs (2jj, 2jj+1); a pair whose first
            // block no query of the wave sees is skipped (its p are 0)
#pragma unroll
            for (int jj = 0; jj < NBW / 2; jj++) {
                if (2 * jj < nvb) {  // wave-uniform
                    const float pv[8] = {p[2 * jj][0],     p[2 * jj][1],     p[2 * jj][2],     p[2 * jj][3],
                                         p[2 * jj + 1][0], p[2 * jj + 1][1], p[2 * jj + 1][2], p[2 * jj + 1][3]};
                    bf16x8 ph, pm;
                    split2(pv, ph, pm);
                    const int key_a = (kg + 2 * jj * KSPLIT) * 16 + 4 * g;        // within the tile
                    const int key_b = (kg + (2 * jj + 1) * KSPLIT) * 16 + 4 * g;
#pragma unroll
                    for (int n = 0; n < NB; n++) {
                        const uint16_t* vr = &v_lds[(16 * n + ql) * VST];
                        bf16x8 vp[2];
#pragma unroll
                        for (int q = 0; q < 2; q++) {
                            const uint2 x0 = *reinterpret_cast<const uint2*>(vr + q * VPLANE + key_a);
                            const uint2 x1 = *reinterpret_cast<const uint2*>(vr + q * VPLANE + key_b);
                            u32x4 t;
                            t[0] = x0.x, t[1] = x0.y, t[2] = x1.x, t[3] = x1.y;
                            vp[q] = __builtin_bit_cast(bf16x8, t);
                        }
                        f32x4 o = acc[n];
                        o = mfma(vp[1], pm, o);
                        o = mfma(vp[1], ph, o);
                        o = mfma(vp[0], pm, o);
                        o = mfma(vp[0], ph, o);
                        acc[n] = o;
                    }
                }
            }
        }
    }

    lsum = sum_over_rows(lsum);
    if constexpr (KSPLIT > 1) {
        __syncthreads();  // every wave is done with the K/V tiles
        float* part = reinterpret_cast<float*>(kv_lds);  // [(KSPLIT-1) x QT sub-tiles][16 queries][HD]
        if (kg > 0) {
            const int slot = (kg - 1) * QT + qs;
            float* o = part + (size_t)slot * 16 * HD + ql * HD;
#pragma unroll
            for (int n = 0; n < NB; n++)
                *reinterpret_cast<float4*>(o + 16 * n + 4 * g) =
                    make_float4(acc[n][0], acc[n][1], acc[n][2], acc[n][3]);
            if (g == 0) {
                s_ml[(slot * 16 + ql) * 2 + 0] = m;
                s_ml[(slot * 16 + ql) * 2 + 1] = lsum;
            }
        }
        __syncthreads();
        if (kg > 0) return;
#pragma unroll
        for (int k = 1; k < KSPLIT; k++) {
            const int slot = (k - 1) * QT + qs;
            const float mo = s_ml[(slot * 16 + ql) * 2 + 0];
            const float lo = s_ml[(slot * 16 + ql) * 2 + 1];
            const float mm = fmaxf(m, mo);
            const float f = scale_of(m, mm), fo = scale_of(mo, mm);
            lsum = lsum * f + lo * fo;
            const float* o = part + (size_t)slot * 16 * HD + ql * HD;
#pragma unroll
            for (int n = 0; n < NB; n++) {
                const float4 t = *reinterpret_cast<const float4*>(o + 16 * n + 4 * g);
                acc[n] = acc[n] * f + f32x4{t.x, t.y, t.z, t.w} * fo;
            }
            m = mm;
        }
    }
    if (row < qcount) {
        const float inv = 1.0f / lsum;
        float* op = a.out + qrow * dim + (size_t)h * HD;
#pragma unroll
        for (int n = 0; n < NB; n++)
            *reinterpret_cast<float4*>(op + 16 * n + 4 * g) =
                make_float4(acc[n][0] * inv, acc[n][1] * inv, acc[n][2] * inv, acc[n][3] * inv);
    }
}

}  // namespace

int prefill_block_m(int) { return BM; }

// hd 128 runs one key group per workgroup (its registers), so 128-row items
// (8 waves, each staged tile serving 128 queries) measured 15-20% faster
// than 64-row ones.  At hd 64 the 64-row items of two key groups are kept:
// 128-row items there need 16-wave workgroups, one per CU, and measured 9%
// slower on the 8-prompt mix (faster on large balanced batches).
bool prefill_uses_wide_items(int32_t kernel, int32_t head_dim) {
    return kernel == PREFILL_KERNEL_DEFAULT && head_dim == 128;
}

bool prefill_appends_in_launch(int32_t kernel, int32_t head_dim, int32_t max_pos, int64_t page_stride) {
    return kernel == PREFILL_KERNEL_DEFAULT && (head_dim == 32 || head_dim == 64 || head_dim == 128) &&
           (max_pos >> 4) < TABLE_LDS && (uint64_t)page_stride * sizeof(float) < (1ull << 32);
}

hipError_t launch_paged_attn_prefill(const PrefillLaunch& a, hipStream_t stream) {
    const dim3 grid((unsigned)((size_t)a.work_items * a.n_heads));
    const bool wide = a.item_rows == PREFILL_WIDE_ROWS;
    if (wide != prefill_uses_wide_items(a.kernel, a.head_dim) || (!wide && a.item_rows != BM))
        return hipErrorInvalidValue;  // the work list must match the kernel's rows per item
    if ((a.k_new != nullptr) != (a.v_new != nullptr) ||
        (a.k_new && !prefill_appends_in_launch(a.kernel, a.head_dim, a.max_pos, a.page_stride)))
        return hipErrorInvalidValue;  // only the bf16 matrix-core kernel appends, with the table in LDS
    if (a.kernel == PREFILL_KERNEL_DEFAULT && a.k_new && !a.append_mixed) {
        switch (a.head_dim) {
            case 32: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<32, 4, 2, 64, 1>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            case 64: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<64, 4, 2, 64, 1>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            case 128: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<128, 8, 1, 32, 1>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            default: return hipErrorInvalidValue;
        }
    }
    if (a.kernel == PREFILL_KERNEL_DEFAULT && a.k_new) {
        switch (a.head_dim) {
            case 32: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<32, 4, 2, 64, 2>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            case 64: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<64, 4, 2, 64, 2>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            case 128: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<128, 8, 1, 32, 2>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            default: return hipErrorInvalidValue;
        }
    }
    if (a.kernel == PREFILL_KERNEL_DEFAULT) {
        switch (a.head_dim) {
            case 32: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<32, 4, 2, 64, 0>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            case 64: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<64, 4, 2, 64, 0>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            case 128: hipLaunchKernelGGL((paged_attn_prefill_x3_kernel<128, 8, 1, 32, 0>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            default: break;  // other head sizes: VALU kernel
        }
    }
    if (a.kernel == PREFILL_KERNEL_MFMA_F32) {
        // 4 query sub-tiles x 2 key groups per workgroup, one workgroup per
        // work item.  (Splitting an item over two workgroups of 2 x 4 balances
        // the schedule better but doubles the K/V each item stages: measured
        // slower, 94 vs 81 us at B=8 x 12 x 64.)
        switch (a.head_dim) {
            case 32: hipLaunchKernelGGL((paged_attn_prefill_mfma_kernel<32, 4, 2, 64>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            case 64: hipLaunchKernelGGL((paged_attn_prefill_mfma_kernel<64, 4, 2, 64>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            case 128: hipLaunchKernelGGL((paged_attn_prefill_mfma_kernel<128, 4, 2, 32>), grid, dim3(512), 0, stream, a); return hipGetLastError();
            default: break;  // other head sizes: VALU kernel
        }
    }
    // VALU kernel: hd 256, head sizes other than 32/64/128/256 (padded), or
    // NITRO_PREFILL_KERNEL=valu
    if (a.head_dim < 4 || a.head_dim > 256 || a.head_dim % 4) return hipErrorInvalidValue;
    const int hdp = a.head_dim <= 32 ? 32 : a.head_dim <= 64 ? 64 : a.head_dim <= 128 ? 128 : 256;
    const bool full = a.head_dim == hdp;
    switch (hdp) {
        case 32:
            if (full) hipLaunchKernelGGL((paged_attn_prefill_kernel<32, true>), grid, dim3(THREADS), 0, stream, a);
            else hipLaunchKernelGGL((paged_attn_prefill_kernel<32, false>), grid, dim3(THREADS), 0, stream, a);
            break;
        case 64:
            if (full) hipLaunchKernelGGL((paged_attn_prefill_kernel<64, true>), grid, dim3(THREADS), 0, stream, a);
            else hipLaunchKernelGGL((paged_attn_prefill_kernel<64, false>), grid, dim3(THREADS), 0, stream, a);
            break;
        case 128:
            if (full) hipLaunchKernelGGL((paged_attn_prefill_kernel<128, true>), grid, dim3(THREADS), 0, stream, a);
            else hipLaunchKernelGGL((paged_attn_prefill_kernel<128, false>), grid, dim3(THREADS), 0, stream, a);
            break;
        default:
            if (full) hipLaunchKernelGGL((paged_attn_prefill_kernel<256, true>), grid, dim3(THREADS), 0, stream, a);
            else hipLaunchKernelGGL((paged_attn_prefill_kernel<256, false>), grid, dim3(THREADS), 0, stream, a);
            break;
    }
    return hipGetLastError();
}

}  // namespace nitro
