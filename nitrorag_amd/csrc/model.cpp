// The transformer step around the attention path: device weights in the
// reference's on-disk layout and the forward passes of src/model_q8.cpp
// (forward_decode_batch :571-694, forward_prefill_chunk :424-557,
// forward_paged :244-368) composed from this library's kernels.  Declared in
// include/nitro_paged_attn.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "capi_common.hpp"
#include "device_pool.hpp"
#include "nitro_paged_attn.h"

using namespace nitro;

struct nitro_model {
    int32_t dim = 0, hidden = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0, vocab = 0, seq_len = 0;
    int32_t head_size = 0, kv_dim = 0;
    uint8_t* weights = nullptr;  // the file's sections after the 28-byte header
    size_t weight_bytes = 0;
    // section offsets (bytes) within `weights`, src/Server_Inference.cpp:52-69
    size_t o_emb = 0, o_rms_att = 0, o_wq = 0, o_wk = 0, o_wv = 0, o_wo = 0, o_rms_ffn = 0;
    size_t o_w1 = 0, o_w2 = 0, o_w3 = 0, o_rms_final = 0, o_freq_real = 0, o_freq_imag = 0;
    // the seven Q8 matrices again in the matrix-core tile layout (Q8Tiled),
    // each section holding every layer (rows are multiples of 16, so no tile
    // spans two layers); read only by products over more than 4 rows of full
    // rows, and built by the first forward that runs one (ensure_tiled)
    uint8_t* tiled = nullptr;
    size_t tiled_bytes = 0;
    size_t t_wq = 0, t_wk = 0, t_wv = 0, t_wo = 0, t_w1 = 0, t_w2 = 0, t_w3 = 0;
    DeviceBuffer<float> x, attn, q, hb, last, ss;
    DeviceBuffer<int32_t> tokens;
    Staging staging;

    const float* f32(size_t off) const { return reinterpret_cast<const float*>(weights + off); }
    const uint8_t* q8(size_t off, int layer, size_t rows, size_t cols) const {
        return weights + off + (size_t)layer * rows * (cols / 32) * 36;
    }
    const uint8_t* q8t(size_t off, int layer, size_t rows, size_t cols) const {
        return tiled ? tiled + off + (size_t)layer * q8_tiled_bytes(rows, cols) : nullptr;
    }
    // (source offset, tiled offset, rows, cols) of each Q8 matrix
    struct Mat {
        size_t src, dst, rows, cols;
    };
    std::vector<Mat> q8_mats() const {
        const size_t D = dim, Hd = hidden, KV = kv_dim;
        return {{o_wq, t_wq, D, D}, {o_wk, t_wk, KV, D}, {o_wv, t_wv, KV, D}, {o_wo, t_wo, D, D},
                {o_w1, t_w1, Hd, D}, {o_w2, t_w2, D, Hd}, {o_w3, t_w3, Hd, D}};
    }
};

namespace {

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Builds the tile-layout copy of the Q8 matrices (1.125 bytes per weight) on
// the first forward that reads it, so a model that never runs more than 4
// rows of full-row products never holds it.  Allocates: a caller capturing
// such forwards into a HIP graph runs one of them before the capture.
void ensure_tiled(nitro_model* m, hipStream_t s) {
    if (m->tiled) return;
    uint8_t* t = nullptr;
    hip_check(hipMalloc((void**)&t, m->tiled_bytes), "hipMalloc(tiled weights)");
    try {
        for (const nitro_model::Mat& mt : m->q8_mats())
            hip_check(launch_q8_tile(m->weights + mt.src, t + mt.dst, (int)(m->n_layers * mt.rows), (int)mt.cols, s),
                      "q8 tile launch");
        // built before any stream reads it, whichever stream a later forward uses
        hip_check(hipStreamSynchronize(s), "q8 tile");
    } catch (...) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(t);
        throw;
    }
    m->tiled = t;
}

void reserve_rows(nitro_model* m, int rows) {
    const size_t r = (size_t)rows;
    m->x.reserve(r * m->dim);
    m->attn.reserve(r * m->dim);
    m->ss.reserve(r * (size_t)((m->dim + 15) / 16));
    m->q.reserve(r * m->dim);
    m->hb.reserve(r * m->hidden);
    m->tokens.reserve(r);
}

void check_model_pool(const nitro_model* m, const nitro_kvpool* pool) {
    require(m != nullptr, ERR_INVALID_ARGUMENT, "null model");
    require(pool != nullptr, ERR_INVALID_ARGUMENT, "null pool");
    require(pool->num_layers == m->n_layers && pool->kv_dim == m->kv_dim, ERR_INVALID_ARGUMENT,
            "pool layers / kv_dim do not match the model");
}

void upload_tokens(nitro_model* m, const int32_t* tokens, int rows, hipStream_t s) {
    require(tokens != nullptr, ERR_INVALID_ARGUMENT, "null tokens");
    for (int i = 0; i < rows; i++)
        if (tokens[i] < 0 || tokens[i] >= m->vocab)
            throw Error(ERR_INVALID_ARGUMENT, "token id " + std::to_string(tokens[i]) + " outside the vocabulary");
    int32_t* h = m->staging.acquire(rows);
    std::memcpy(h, tokens, sizeof(int32_t) * rows);
    m->staging.copy(m->tokens.ptr, h, rows, s);
    m->staging.finish(s);
}

// logits = wcls . rms_norm(x) for `rows` rows of the residual stream x, which
// are rows first .. first + rows - 1 of the `total` rows the last residual
// product left partial sums of squares for (src/model_q8.cpp:553-555,
// :687-692).  The norm rides in the classifier launch where its flat kernel
// takes the batch (x stays unnormalised); otherwise x is normalised in place
// first.
void final_logits(nitro_model* m, float* x, int first, int total, int rows, float* logits, hipStream_t s) {
    const Q8Norm nm{m->f32(m->o_rms_final), m->ss.ptr + first, (m->dim + 15) / 16, total};
    if (launch_f32_matmul_norm(m->f32(m->o_emb), x, nm, logits, rows, m->dim, m->vocab, s)) {
        hip_check(hipGetLastError(), "classifier launch");
        return;
    }
    hip_check(launch_add_rmsnorm(x, nullptr, m->f32(m->o_rms_final), x, rows, m->dim, s), "rmsnorm launch");
    hip_check(launch_f32_matmul(m->f32(m->o_emb), x, logits, rows, m->dim, m->vocab, s), "classifier launch");
}

// The layer loop shared by the decode, prefill and mixed forwards.  x is the
// residual stream; rms_norm is folded into the products that read it (wq/wk/wv
// and w1/w3 take rms_norm(x, rms_att / rms_ffn) as input), and wo and w2 add
// their products into x in place, leaving per row the partial sums of
// squares the next norm needs in `ss` (src/model_q8.cpp:584-684).  After it x
// holds the final residual stream.
template <typename Attend>
void layers(nitro_model* m, nitro_kvpool* pool, const int32_t* tokens, int rows, int semantics, Q8Rope rope,
            hipStream_t s, Attend attend) {
    const int dim = m->dim, kv = m->kv_dim, hid = m->hidden;
    const bool last = semantics == NITRO_Q8_LAST_BLOCK;
    const int parts = (dim + 15) / 16;  // partials per row left by wo / w2
    if (!last && rows > Q8_GEMV_MAX_BATCH) ensure_tiled(m, s);
    hip_check(launch_embed_rows(m->f32(m->o_emb), tokens, m->x.ptr, rows, dim, m->vocab, pool->bad_pages.ptr,
                                m->ss.ptr, s),
              "embed launch");
    for (int l = 0; l < m->n_layers; l++) {
        // q, k, v = wq/wk/wv . rms_norm(x, rms_att) in one launch, RoPE on q and
        // k, k and v appended to the pools (:586-617)
        const Q8Norm att{m->f32(m->o_rms_att) + (size_t)l * dim, m->ss.ptr, l ? parts : 1, rows};
        const void* wqkv[3] = {m->q8(m->o_wq, l, dim, dim), m->q8(m->o_wk, l, kv, dim),
                               m->q8(m->o_wv, l, kv, dim)};
        Q8Tiled tqkv;
        tqkv.w[0] = m->q8t(m->t_wq, l, dim, dim);
        tqkv.w[1] = m->q8t(m->t_wk, l, kv, dim);
        tqkv.w[2] = m->q8t(m->t_wv, l, kv, dim);
        const int dqkv[3] = {dim, kv, kv};
        rope.layer_off = pool->layer_offset(l);
        hip_check(launch_q8_qkv(wqkv, m->x.ptr, m->q.ptr, dqkv, rows, dim, last, att, rope, s, tqkv),
                  "q8_qkv launch");
        attend(l);  // attention over the pools -> m->attn (:618-662)
        // x += wo . attn (:663-666)
        hip_check(launch_q8_residual(m->q8(m->o_wo, l, dim, dim), m->attn.ptr, m->x.ptr, m->ss.ptr, rows, dim,
                                     dim, last, s, m->q8t(m->t_wo, l, dim, dim)),
                  "q8 wo launch");
        // hb = silu(w1 . xb) * (w3 . xb), xb = rms_norm(x, rms_ffn), one launch (:667-680)
        const Q8Norm ffn{m->f32(m->o_rms_ffn) + (size_t)l * dim, m->ss.ptr, parts, rows};
        Q8Tiled t13;
        t13.w[0] = m->q8t(m->t_w1, l, hid, dim);
        t13.w[1] = m->q8t(m->t_w3, l, hid, dim);
        hip_check(launch_q8_swiglu(m->q8(m->o_w1, l, hid, dim), m->q8(m->o_w3, l, hid, dim), m->x.ptr,
                                   m->hb.ptr, rows, dim, hid, last, ffn, s, t13),
                  "q8_swiglu launch");
        // x += w2 . hb (:682-684)
        hip_check(launch_q8_residual(m->q8(m->o_w2, l, dim, hid), m->hb.ptr, m->x.ptr, m->ss.ptr, rows, hid,
                                     dim, last, s, m->q8t(m->t_w2, l, dim, hid)),
                  "q8 w2 launch");
    }
}

size_t q8_bytes(size_t rows, size_t cols) { return rows * (cols / 32) * 36; }

// RoPE / K-V append arguments of a forward: rows below `split` take position
// and slot from (pos_a, slot_a), the rest from (pos_b, slot_b).
Q8Rope rope_args(const nitro_model* m, nitro_kvpool* pool, const int32_t* pos_a, const int32_t* slot_a,
                 int split, const int32_t* pos_b, const int32_t* slot_b) {
    Q8Rope r;
    r.freq_real = m->f32(m->o_freq_real);
    r.freq_imag = m->f32(m->o_freq_imag);
    r.head_dim = m->head_size;
    r.k_pool = pool->k;
    r.v_pool = pool->v;
    r.page_stride = pool->page_stride();
    r.num_pages = pool->num_pages;
    r.bad_pages = pool->bad_pages.ptr;
    r.pos[0] = pos_a;
    r.slot[0] = slot_a;
    r.pos[1] = pos_b;
    r.slot[1] = slot_b;
    r.split = split;
    return r;
}

void check_positions(const nitro_model* m, int max_pos) {
    if (max_pos >= m->seq_len)
        throw Error(ERR_INVALID_ARGUMENT, "position " + std::to_string(max_pos) + " is outside the model's seq_len");
}

int max_of(const std::vector<int32_t>& v) {
    int r = 0;
    for (int x : v) r = std::max(r, (int)x);
    return r;
}

}  // namespace

namespace nitro {

void model_dims(const nitro_model* m, int32_t* dims) {
    dims[0] = m->dim;
    dims[1] = m->vocab;
    dims[2] = m->seq_len;
    dims[3] = m->n_layers;
    dims[4] = m->kv_dim;
}

void forward_mixed(nitro_model* m, nitro_kvpool* pool, const int32_t* tokens, int P, int B,
                   bool prefill_as_decode, bool prefill_logits, float* logits, int32_t* next, int semantics,
                   hipStream_t s) {
    check_model_pool(m, pool);
    require(P >= 0 && B >= 0 && P + B > 0, ERR_INVALID_ARGUMENT, "no rows");
    require(!prefill_logits || P > 0, ERR_INVALID_ARGUMENT, "prefill logits without prefill rows");
    if (prefill_as_decode) {
        require(pool->decode.batch == P + B, ERR_NO_BATCH, "the rows differ from the decode batch");
    } else {
        require(P == 0 || (pool->prefill.batch == 1 && pool->prefill.total_rows == P), ERR_NO_BATCH,
                "the prefill rows differ from the uploaded one-sequence prefill batch");
        require(B == 0 || pool->decode.batch == B, ERR_NO_BATCH, "the decode rows differ from the decode batch");
    }
    const size_t dim = m->dim;
    void* stream = s;
    const DecodeBatch& d = pool->decode;
    const PrefillBatch& pf = pool->prefill;
    if (prefill_as_decode || B > 0) check_positions(m, max_of(d.positions));
    if (!prefill_as_decode && P > 0) check_positions(m, pf.max_pos);
    // every row's RoPE position and K/V slot: the decode batch's, or the
    // prefill batch's for rows [0, P) when those go through the prefill kernel
    const Q8Rope rope = prefill_as_decode || P == 0
                            ? rope_args(m, pool, d.pos.ptr, d.slots.ptr, P + B, nullptr, nullptr)
                            : rope_args(m, pool, pf.row_pos.ptr, pf.slots.ptr, P, d.pos.ptr, d.slots.ptr);
    reserve_rows(m, P + B);
    layers(m, pool, tokens, P + B, semantics, rope, s, [&](int l) {
        if (prefill_as_decode) {
            // every row attends its own prefix (keys 0..position) in one
            // decode-attention launch; a chunk row at position p sees the same
            // keys as in forward_prefill_chunk (src/model_q8.cpp:493-530)
            require(nitro_paged_attn_decode(pool, l, m->q.ptr, m->attn.ptr, m->n_heads, m->n_kv_heads,
                                            m->head_size, stream) == NITRO_OK,
                    ERR_INVALID_ARGUMENT, nitro_last_error());
            return;
        }
        // forward_prefill_chunk's causal attention for rows [0, P)
        // (src/model_q8.cpp:471-530), forward_decode_batch's for the rest (:618-662)
        if (P > 0)
            require(nitro_paged_attn_prefill(pool, l, m->q.ptr, m->attn.ptr, m->n_heads, m->n_kv_heads,
                                             m->head_size, stream) == NITRO_OK,
                    ERR_INVALID_ARGUMENT, nitro_last_error());
        if (B > 0)
            require(nitro_paged_attn_decode(pool, l, m->q.ptr + P * dim, m->attn.ptr + P * dim, m->n_heads,
                                            m->n_kv_heads, m->head_size, stream) == NITRO_OK,
                    ERR_INVALID_ARGUMENT, nitro_last_error());
    });
    // The rows whose logits are used are contiguous: the chunk's last row
    // (when it completes its prompt) and the decode rows.  rms_norm; logits =
    // wcls . x (:553-555, :687-692); argmax (:559-569).
    const int first = prefill_logits ? P - 1 : P;
    const int out_rows = P + B - first;
    if (out_rows == 0) return;
    float* x = m->x.ptr + first * dim;
    final_logits(m, x, first, P + B, out_rows, logits, s);
    hip_check(launch_argmax_rows(logits, next, out_rows, m->vocab, s), "argmax launch");
    pool->last_stream = s;
}

}  // namespace nitro

extern "C" {

int nitro_model_create(const void* blob, uint64_t bytes, nitro_model** out) {
    return guarded([&] {
        require(out != nullptr, ERR_INVALID_ARGUMENT, "null output pointer");
        *out = nullptr;
        require(blob != nullptr && bytes >= 28, ERR_INVALID_ARGUMENT, "model blob shorter than its header");
        int32_t h[7];
        std::memcpy(h, blob, sizeof(h));
        nitro_model* m = new nitro_model();
        try {
            m->dim = h[0];
            m->hidden = h[1];
            m->n_layers = h[2];
            m->n_heads = h[3];
            m->n_kv_heads = h[4];
            m->vocab = h[5];
            m->seq_len = h[6];
            require(m->dim > 0 && m->hidden > 0 && m->n_layers > 0 && m->n_heads > 0 &&
                        m->n_kv_heads > 0 && m->vocab > 0 && m->seq_len > 0,
                    ERR_INVALID_ARGUMENT, "header fields must be positive");
            require(m->dim % m->n_heads == 0 && m->n_heads % m->n_kv_heads == 0, ERR_UNSUPPORTED,
                    "dim must split into heads and heads into KV groups");
            m->head_size = m->dim / m->n_heads;
            m->kv_dim = m->n_kv_heads * m->head_size;
            require(attention_head_dim(m->head_size), ERR_UNSUPPORTED,
                    "head_size must be a multiple of 4 from 4 to 256");
            require(m->dim % 64 == 0 && m->hidden % 32 == 0 && m->kv_dim % 32 == 0, ERR_UNSUPPORTED,
                    "dim must be a multiple of 64, hidden_dim and kv_dim of 32");
            const size_t L = m->n_layers, D = m->dim, Hd = m->hidden, KV = m->kv_dim, V = m->vocab;
            size_t o = 0;
            m->o_emb = o;        o += V * D * 4;
            m->o_rms_att = o;    o += L * D * 4;
            m->o_wq = o;         o += L * q8_bytes(D, D);
            m->o_wk = o;         o += L * q8_bytes(KV, D);
            m->o_wv = o;         o += L * q8_bytes(KV, D);
            m->o_wo = o;         o += L * q8_bytes(D, D);
            m->o_rms_ffn = o;    o += L * D * 4;
            m->o_w1 = o;         o += L * q8_bytes(Hd, D);
            m->o_w2 = o;         o += L * q8_bytes(D, Hd);
            m->o_w3 = o;         o += L * q8_bytes(Hd, D);
            m->o_rms_final = o;  o += D * 4;
            m->o_freq_real = o;  o += (size_t)m->seq_len * m->head_size / 2 * 4;
            m->o_freq_imag = o;  o += (size_t)m->seq_len * m->head_size / 2 * 4;
            if (bytes < 28 + o)
                throw Error(ERR_INVALID_ARGUMENT, "model blob holds " + std::to_string(bytes) +
                                                      " bytes; its header needs " + std::to_string(28 + o));
            m->weight_bytes = o;
            hip_check(hipMalloc((void**)&m->weights, o), "hipMalloc(weights)");
            hip_check(hipMemcpy(m->weights, static_cast<const uint8_t*>(blob) + 28, o, hipMemcpyHostToDevice),
                      "hipMemcpy(weights)");
            // offsets of the tile-layout copies (built by the first forward that
            // reads them), all layers of a matrix together
            size_t t = 0;
            size_t* dst[7] = {&m->t_wq, &m->t_wk, &m->t_wv, &m->t_wo, &m->t_w1, &m->t_w2, &m->t_w3};
            const std::vector<nitro_model::Mat> mats = m->q8_mats();
            for (int i = 0; i < 7; i++) {
                *dst[i] = t;
                t += L * q8_tiled_bytes(mats[i].rows, mats[i].cols);
            }
            m->tiled_bytes = t;
        } catch (...) {
            if (m->tiled) (void)hipFree(m->tiled);
            if (m->weights) (void)hipFree(m->weights);
            delete m;
            throw;
        }
        *out = m;
    });
}

int nitro_model_destroy(nitro_model* m) {
    if (!m) return NITRO_OK;
    return guarded([&] {
        (void)hipDeviceSynchronize();
        (void)hipFree(m->weights);
        (void)hipFree(m->tiled);
        delete m;
    });
}

int nitro_model_config(const nitro_model* m, int32_t* cfg) {
    return guarded([&] {
        require(m != nullptr && cfg != nullptr, ERR_INVALID_ARGUMENT, "null pointer");
        const int32_t v[7] = {m->dim, m->hidden, m->n_layers, m->n_heads, m->n_kv_heads, m->vocab, m->seq_len};
        std::memcpy(cfg, v, sizeof(v));
    });
}

int nitro_forward_decode_batch(nitro_model* m, nitro_kvpool* pool, const int32_t* tokens, int32_t batch,
                               float* logits, int32_t semantics, void* stream) {
    return guarded([&] {
        check_model_pool(m, pool);
        require(logits != nullptr, ERR_INVALID_ARGUMENT, "null logits");
        require(semantics == NITRO_Q8_FULL_ROWS || semantics == NITRO_Q8_LAST_BLOCK, ERR_INVALID_ARGUMENT,
                "unknown Q8 semantics");
        require(pool->decode.batch > 0, ERR_NO_BATCH, "no decode batch uploaded");
        require(batch == pool->decode.batch, ERR_INVALID_ARGUMENT,
                "batch differs from the uploaded decode batch");
        hipStream_t s = as_stream(stream);
        const DecodeBatch& d = pool->decode;
        check_positions(m, max_of(d.positions));
        reserve_rows(m, batch);
        upload_tokens(m, tokens, batch, s);
        const Q8Rope rope = rope_args(m, pool, d.pos.ptr, d.slots.ptr, batch, nullptr, nullptr);
        layers(m, pool, m->tokens.ptr, batch, semantics, rope, s, [&](int l) {
            require(nitro_paged_attn_decode(pool, l, m->q.ptr, m->attn.ptr, m->n_heads, m->n_kv_heads,
                                            m->head_size, stream) == NITRO_OK,
                    ERR_INVALID_ARGUMENT, nitro_last_error());
        });
        // logits = wcls . rms_norm(x) (:687-692)
        final_logits(m, m->x.ptr, 0, batch, batch, logits, s);
        pool->last_stream = s;
    });
}

int nitro_forward_prefill(nitro_model* m, nitro_kvpool* pool, const int32_t* tokens, int32_t total_rows,
                          float* logits, int32_t semantics, void* stream) {
    return guarded([&] {
        check_model_pool(m, pool);
        require(logits != nullptr, ERR_INVALID_ARGUMENT, "null logits");
        require(semantics == NITRO_Q8_FULL_ROWS || semantics == NITRO_Q8_LAST_BLOCK, ERR_INVALID_ARGUMENT,
                "unknown Q8 semantics");
        const PrefillBatch& p = pool->prefill;
        require(p.batch > 0, ERR_NO_BATCH, "no prefill batch uploaded");
        require(total_rows == p.total_rows, ERR_INVALID_ARGUMENT,
                "total_rows differs from the uploaded prefill batch");
        hipStream_t s = as_stream(stream);
        reserve_rows(m, total_rows);
        m->last.reserve((size_t)p.batch * m->dim);
        upload_tokens(m, tokens, total_rows, s);
        check_positions(m, p.max_pos);
        const Q8Rope rope = rope_args(m, pool, p.row_pos.ptr, p.slots.ptr, total_rows, nullptr, nullptr);
        layers(m, pool, m->tokens.ptr, total_rows, semantics, rope, s, [&](int l) {
            require(nitro_paged_attn_prefill(pool, l, m->q.ptr, m->attn.ptr, m->n_heads, m->n_kv_heads,
                                             m->head_size, stream) == NITRO_OK,
                    ERR_INVALID_ARGUMENT, nitro_last_error());
        });
        // Each chunk's last token: rms_norm; logits = wcls . x (:553-555)
        hip_check(launch_gather_last_rows(m->x.ptr, nullptr, p.d_row_off.ptr, p.d_len.ptr, m->last.ptr,
                                          p.batch, m->dim, s),
                  "gather launch");
        hip_check(launch_add_rmsnorm(m->last.ptr, nullptr, m->f32(m->o_rms_final), m->last.ptr, p.batch,
                                     m->dim, s),
                  "rmsnorm launch");
        hip_check(launch_f32_matmul(m->f32(m->o_emb), m->last.ptr, logits, p.batch, m->dim, m->vocab, s),
                  "classifier launch");
        pool->last_stream = s;
    });
}

}  // extern "C"
