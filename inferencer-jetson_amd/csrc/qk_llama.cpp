// qk_llama.cpp - Llama decode-step driver over the qk C ABI.
//
// The counterpart of FastGPU / FastRunner (inferencer.cu:1101-1150,
// 1182-1532): buffers, KV cache and RoPE tables are allocated once in
// qk_llama_create; qk_llama_forward issues one step with the arithmetic of
// FastRunner::forward (inferencer.cu:1424-1531) in five launches per layer:
// the RMSNorms, SiLU * up and residual adds are fused into the GEMVs around
// them, RoPE and the KV write into the attention kernel.  The step is generalised
// past the reference's Llama-3.2-3B hard-coding (inferencer.cu:1215-1217):
// any head_dim dividing 256, GQA group and layer count.
//
// The greedy token of a step stays on the device; when the caller feeds it
// back as the next input token the embedding reads it there, so a decode
// loop moves 4 bytes device->host per token (the reference's copy,
// inferencer.cu:1529) and nothing host->device.
#include "qk_internal.h"

#include <algorithm>
#include <cmath>
#include <vector>

struct qk_llama {
    qk_llama_config cfg{};
    qk_llama_weights w{};
    std::vector<qk_llama_layer> layers;
    hipStream_t stream = nullptr;
    int head_dim = 0, kv_dim = 0;
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    float *attn = nullptr, *tmp = nullptr, *gate = nullptr, *up = nullptr, *logits = nullptr;
    float *key_cache = nullptr, *value_cache = nullptr, *cosine = nullptr, *sine = nullptr;
    void *argmax_ws = nullptr;
    void *attn_ws = nullptr;   // split-attention partials
    size_t attn_ws_bytes = 0;
    int32_t *d_next = nullptr, *d_token = nullptr;
    int32_t *h_token = nullptr;   // pinned staging for host tokens and the result
    // The greedy token as the final pick writes it into host-coherent pinned
    // memory (h_next; hd_next its device address): the host reads it once
    // the stream is done, with no download launch.  next_mirrored: this
    // step's pick wrote it.
    int32_t *h_next = nullptr, *hd_next = nullptr;
    bool next_mirrored = false;
    // INT8 steps: the final pick also writes the picked token's embedding
    // row into x_next; the next step, fed that token, swaps x_next in as x
    // instead of launching the embedding (x keeps the residual stream until
    // then, as qk_llama_residual reports it).
    float *x_next = nullptr;
    bool x_next_valid = false;
    hipEvent_t upload_done = nullptr;   // the last token upload from h_token[0] has read it
    bool upload_pending = false;
    int last_next = -1;
    int int8_q4k = 0, int8_q6k = 0;            // INT8 GEMV mode (use_dp4a / use_q6_dp4a)
    int8_t *xq = nullptr;                      // INT8 mode: quantized activations, max(dim, hidden)
    float *xscale = nullptr;
    // FP32 step over activation records (records = true): each GEMV reads the
    // records its producer made -- x * attn_norm for QKV (rec_norm, made by
    // the embedding or the previous down projection; x * output_norm for the
    // LM head), the attention output for o (rec_attn), x * ffn_norm for
    // gate/up (rec_ffn, made by o), SiLU(gate) * up for down (rec_silu) --
    // with the sums of squares of x for the RMSNorms (ss_norm, ss_ffn).
    bool records = false;
    qk::XGroup *rec_norm = nullptr, *rec_attn = nullptr, *rec_ffn = nullptr, *rec_silu = nullptr;
    float *ss_norm = nullptr, *ss_ffn = nullptr;
    std::vector<void *> owned;    // split-layout copies of the Q6_K weights
    qk_llama_memory mem{};        // device bytes the handle holds
    uint64_t matrix_calls = 0;    // quantized matrix products issued (FastGPU::calls)
    // qk_llama_set_trace: the residual after each layer [layer][dim] and the
    // INT8 inputs of each layer's products [layer][4][max(dim, hidden)].
    float *trace_x = nullptr;
    int8_t *trace_q = nullptr;
};

namespace {

// Trace copies of a step (device to device, on the step's stream).
int trace_copy(void *dst, const void *src, size_t bytes, hipStream_t s) {
    if (!dst) return QK_OK;
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s) != hipSuccess)
        return qk::fail(QK_ERR_DEVICE, "trace copy failed");
    return QK_OK;
}

// The same for the rows of a batch: rows of `width` bytes `spitch` apart
// into rows `dpitch` apart.
int trace_copy_2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width, int rows, hipStream_t s) {
    if (!dst) return QK_OK;
    if (hipMemcpy2DAsync(dst, dpitch, src, spitch, width, rows, hipMemcpyDeviceToDevice, s) != hipSuccess)
        return qk::fail(QK_ERR_DEVICE, "trace copy failed");
    return QK_OK;
}

template <class T>
int dev_alloc(uint64_t &total, T **p, size_t count, const char *what) {
    if (hipMalloc(reinterpret_cast<void **>(p), count * sizeof(T)) != hipSuccess)
        return qk::fail(QK_ERR_DEVICE, std::string("qk_llama_create: cannot allocate ") + what);
    total += count * sizeof(T);
    return QK_OK;
}

void release(qk_llama *m) {
    void *bufs[] = {m->x, m->x_next, m->xn, m->q, m->k, m->v, m->attn, m->tmp, m->gate, m->up, m->logits, m->key_cache,
                    m->value_cache, m->cosine, m->sine, m->argmax_ws, m->attn_ws, m->d_next, m->d_token,
                    m->xq, m->xscale, m->rec_norm, m->rec_attn, m->rec_ffn, m->rec_silu, m->ss_norm, m->ss_ffn};
    for (void *b : bufs)
        if (b) (void)hipFree(b);
    if (m->h_token) (void)hipHostFree(m->h_token);
    if (m->h_next) (void)hipHostFree(m->h_next);
    if (m->upload_done) (void)hipEventDestroy(m->upload_done);
    for (void *b : m->owned) (void)hipFree(b);
    delete m;
}

bool quant_type(int t) { return t == QK_TYPE_Q4_K || t == QK_TYPE_Q6_K || t == QK_TYPE_Q6_K_SPLIT; }

// A Q6_K tensor in the GGUF layout is copied once into the split layout
// (QK_TYPE_Q6_K_SPLIT: every field a kernel reads 16-byte aligned) and the
// driver uses the copy; the caller keeps its weights.
int split_tensor(std::vector<void *> &owned, uint64_t &total, int &type, const void *&w, int cols, int rows,
                 hipStream_t s) {
    if (type != QK_TYPE_Q6_K) return QK_OK;
    void *dst = nullptr;
    const size_t bytes = static_cast<size_t>(qk_tensor_bytes(QK_TYPE_Q6_K_SPLIT, cols, rows));
    if (hipMalloc(&dst, bytes) != hipSuccess) return qk::fail(QK_ERR_DEVICE, "cannot allocate a split-layout Q6_K copy");
    owned.push_back(dst);
    total += bytes;
    if (int st = qk_q6k_split(w, dst, cols, rows, s)) return st;
    type = QK_TYPE_Q6_K_SPLIT;
    w = dst;
    return QK_OK;
}

int split_weights(std::vector<void *> &owned, uint64_t &total, qk_llama_weights &w,
                  std::vector<qk_llama_layer> &layers, const qk_llama_config &c, int kv_dim, hipStream_t s) {
    int st;
    for (qk_llama_layer &L : layers)
        if ((st = split_tensor(owned, total, L.q_type, L.q, c.dim, c.dim, s)) ||
            (st = split_tensor(owned, total, L.k_type, L.k, c.dim, kv_dim, s)) ||
            (st = split_tensor(owned, total, L.v_type, L.v, c.dim, kv_dim, s)) ||
            (st = split_tensor(owned, total, L.o_type, L.o, c.dim, c.dim, s)) ||
            (st = split_tensor(owned, total, L.gate_type, L.gate, c.dim, c.hidden, s)) ||
            (st = split_tensor(owned, total, L.up_type, L.up, c.dim, c.hidden, s)) ||
            (st = split_tensor(owned, total, L.down_type, L.down, c.hidden, c.dim, s)))
            return st;
    if ((st = split_tensor(owned, total, w.embd_type, w.token_embd, c.dim, c.vocab, s))) return st;
    if (w.output && (st = split_tensor(owned, total, w.output_type, w.output, c.dim, c.vocab, s))) return st;
    // The copies are complete before create returns: the caller may release
    // its Q6_K buffers from then on.
    if (hipStreamSynchronize(s) != hipSuccess) return qk::fail(QK_ERR_DEVICE, "Q6_K split copies failed");
    return QK_OK;
}

// Bytes of the split-layout copies create makes (every GGUF-layout Q6_K tensor).
uint64_t split_copy_bytes(const qk_llama_weights &w, const qk_llama_config &c, int kv_dim) {
    auto one = [](int type, int cols, int rows) -> uint64_t {
        return type == QK_TYPE_Q6_K ? static_cast<uint64_t>(qk_tensor_bytes(QK_TYPE_Q6_K_SPLIT, cols, rows)) : 0;
    };
    uint64_t b = one(w.embd_type, c.dim, c.vocab) + (w.output ? one(w.output_type, c.dim, c.vocab) : 0);
    for (int l = 0; l < c.layers; ++l) {
        const qk_llama_layer &L = w.layers[l];
        b += one(L.q_type, c.dim, c.dim) + one(L.k_type, c.dim, kv_dim) + one(L.v_type, c.dim, kv_dim) +
             one(L.o_type, c.dim, c.dim) + one(L.gate_type, c.dim, c.hidden) + one(L.up_type, c.dim, c.hidden) +
             one(L.down_type, c.hidden, c.dim);
    }
    return b;
}

// The reference's upload check (inferencer.cu:329-333): the device must have
// the bytes about to be allocated plus a 64 MiB margin free.
int check_free_memory(const char *where, uint64_t need) {
    size_t free_bytes = 0, total_bytes = 0;
    if (hipMemGetInfo(&free_bytes, &total_bytes) != hipSuccess)
        return qk::fail(QK_ERR_DEVICE, std::string(where) + ": device memory query failed");
    if (free_bytes < need + (uint64_t(64) << 20))
        return qk::fail(QK_ERR_DEVICE, std::string(where) + ": not enough free device memory (" +
                                           std::to_string(need) + " bytes needed for caches, buffers and "
                                           "split Q6_K copies, " + std::to_string(free_bytes) + " free)");
    return QK_OK;
}

bool int8_type(const qk_llama *m, int type) {
    return (type == QK_TYPE_Q4_K && m->int8_q4k) ||
           ((type == QK_TYPE_Q6_K || type == QK_TYPE_Q6_K_SPLIT) && m->int8_q6k);
}

// y_m = W_m x for each matrix: the INT8 kernels on m->xq / m->xscale (already
// quantized from x) for the types in INT8 mode, the FP32 kernels on x for the
// others -- FastGPU::matvec's per-type choice (inferencer.cu:1159-1168) and
// qkv_cuda's per-row branch (inferencer.cu:776-780).
// Matrices in FP32 mode cannot add into y (the plain kernels overwrite), so
// callers pass accumulate only for a single INT8 matrix.
int gemv_by_mode(qk_llama *m, const qk_matrix *mats, int n, const float *x, int cols, hipStream_t s,
                 int accumulate = 0) {
    qk_matrix i8[QK_MAX_FUSED], f32[QK_MAX_FUSED];
    int ni = 0, nf = 0, st;
    for (int k = 0; k < n; ++k) (int8_type(m, mats[k].type) ? i8[ni++] : f32[nf++]) = mats[k];
    if (ni && (st = qk::launch_gemv_i8(i8, ni, m->xq, cols, m->xscale, cols / 32, cols, 1, nullptr, accumulate, s)))
        return st;
    if (nf && (st = qk::launch_gemv_f32(f32, nf, x, cols, cols, 1, nullptr, s))) return st;
    return QK_OK;
}

// x += W in for the o / down projections, the sum add_cuda forms
// (inferencer.cu:1464, 1507): an INT8 matrix adds in its own epilogue
// (y = x, accumulate), an FP32 one in the fused kernel's residual epilogue;
// rows too long to stage write tmp and a separate add follows.
int residual_by_mode(qk_llama *m, int type, int rows, const void *w, const float *in, int cols, hipStream_t s) {
    int st;
    if (int8_type(m, type)) {
        const qk_matrix mat{type, rows, w, m->x};
        return gemv_by_mode(m, &mat, 1, in, cols, s, 1);
    }
    if (qk::gemv_fusable(cols)) {
        qk::GemvFusion residual;
        residual.accumulate = 1;
        const qk_matrix mat{type, rows, w, m->x};
        return qk::launch_gemv_fused(&mat, 1, in, cols, cols, 1, nullptr, residual, s);
    }
    const qk_matrix mat{type, rows, w, m->tmp};
    if ((st = gemv_by_mode(m, &mat, 1, in, cols, s))) return st;
    return qk_add_f32(m->x, m->tmp, rows, s);
}

// Rows per split of the one-sequence attention when the o GEMV merges its
// splits: one round of the wide kernel's rows (128 at head_dim 64) per
// workgroup, longer when that would take more than the 8 splits the merging
// GEMVs hold.
int decode_split_rows(int rows) { return std::max(128, ((rows + 7) / 8 + 15) / 16 * 16); }

// The INT8 mode of FastRunner::forward (inferencer.cu:1424-1531 with use_dp4a /
// use_q6_dp4a and --fused-norm-quant): RMSNorm and the per-32 quantization in
// one launch before the QKV and gate/up GEMVs, the attention output quantized
// before the o GEMV, SiLU * up and its quantization in one launch before the
// down GEMV, and the residual adds in the INT8 GEMVs' epilogues (the same
// fp32 sums as the reference's separate add launches).  With every matrix in
// INT8 mode and no input traces, the QKV and gate/up GEMVs quantize their
// own inputs instead (launch_gemv_i8_staged) and the attention quantizes
// o's: the same codes, three launches per layer fewer.
int forward_int8(qk_llama *m, const int32_t *tok, int pos, bool need_logits, bool embedded, hipStream_t s) {
    const qk_llama_config &c = m->cfg;
    const int dim = c.dim, kv = m->kv_dim, hd = m->head_dim;
    int st;
    const bool staged = m->int8_q4k && m->int8_q6k && !m->trace_q && qk::gemv_i8_stageable(dim);
    const bool q8 = c.heads * hd == dim && hd % 32 == 0;   // the attention can quantize o's input
    // With both modes on, the attention's rows split into rounds of 128 per
    // workgroup (at most 8 splits) and the o GEMV merges the splits while it
    // stages its input (launch_gemv_i8_merged): the attention's CUs each
    // stream one round of rows instead of all of a head's.  The traced step
    // takes the same splits, merged by the merge kernel, so its codes are
    // the staged step's.
    const bool merge_o = m->int8_q4k && m->int8_q6k && q8 && qk::gemv_i8_stageable(dim) &&
                         qk::gemv_i8_mergeable(dim, hd, 8);
    if (embedded)
        std::swap(m->x, m->x_next);   // the previous pick wrote this token's row
    else if ((st = qk_embedding(m->w.embd_type, m->w.token_embd, tok, 1, m->x, dim, c.vocab, s)))
        return st;
    qk::SplitAttention attn{};
    attn.wide_split_rows = merge_o ? decode_split_rows(pos + 1) : 0;
    attn.q = m->q;
    attn.k = m->k;
    attn.v = m->v;
    attn.cosine = m->cosine;
    attn.sine = m->sine;
    attn.key_cache = m->key_cache;
    attn.head_major = 1;
    attn.value_cache = m->value_cache;
    attn.out = m->attn;
    attn.cache_rows = c.context;
    attn.rows_hint = pos + 1;
    attn.pos = attn.max_pos = pos;
    attn.n_tokens = 1;
    attn.heads = c.heads;
    attn.kv_heads = c.kv_heads;
    attn.head_dim = hd;
    auto norm_quant = [&](const float *w) {
        return qk_rmsnorm_quantize_x32(m->x, dim, w, m->xn, dim, m->xq, dim, m->xscale, dim / 32, dim, 1, c.eps, s);
    };
    const size_t qstride = std::max(dim, c.hidden);
    auto trace_q = [&](int l, int stage, int cols) {
        return trace_copy(m->trace_q ? m->trace_q + (l * 4 + stage) * qstride : nullptr, m->xq, cols, s);
    };
    for (int l = 0; l < c.layers && staged; ++l) {
        const qk_llama_layer &L = m->layers[l];
        const qk_matrix qkv[3] = {{L.q_type, dim, L.q, m->q}, {L.k_type, kv, L.k, m->k}, {L.v_type, kv, L.v, m->v}};
        if ((st = qk::launch_gemv_i8_staged(qkv, 3, m->x, dim, L.attn_norm, c.eps, nullptr, dim, 1, nullptr, 0, s)))
            return st;
        attn.layer = l;
        attn.q8_out = q8 ? m->xq : nullptr;
        attn.q8_scale = q8 ? m->xscale : nullptr;
        attn.defer_merge = merge_o;
        int parts = 1;   // splits left for o to merge
        if ((st = qk::launch_split_attention(attn, 0, m->attn_ws, m->attn_ws_bytes, s, &parts))) return st;
        const qk_matrix o{L.o_type, dim, L.o, m->x};
        const qk_matrix gu[2] = {{L.gate_type, c.hidden, L.gate, m->gate}, {L.up_type, c.hidden, L.up, m->up}};
        const qk_matrix down{L.down_type, dim, L.down, m->x};
        const bool pair = L.gate_type == L.up_type && qk::gemv_i8_pair_supported(dim, c.hidden);
        // o merges the attention's splits, or reads the codes the attention
        // wrote, or quantizes the attention's output itself; the gate / up pair quantizes SiLU(gate) * up for
        // down in its epilogue when both are one type; down keeps its own
        // launch (staging SiLU * up would read and activate the whole
        // 4 x hidden bytes in every workgroup).
        if ((st = parts > 1 ? qk::launch_gemv_i8_merged(&o, 1, static_cast<const float *>(m->attn_ws), parts, hd, dim,
                                                         1, s)
                  : q8      ? qk::launch_gemv_i8(&o, 1, m->xq, dim, m->xscale, dim / 32, dim, 1, nullptr, 1, s)
                            : qk::launch_gemv_i8_staged(&o, 1, m->attn, dim, nullptr, 0.f, nullptr, dim, 1, nullptr, 1,
                                                        s)) ||
            (st = pair ? qk::launch_gemv_i8_pair_quant(gu, m->x, dim, L.ffn_norm, c.eps, dim, 1, m->xq, m->xscale,
                                                       c.hidden, c.hidden / 32, s)
                       : qk::launch_gemv_i8_staged(gu, 2, m->x, dim, L.ffn_norm, c.eps, nullptr, dim, 1, nullptr, 0,
                                                   s)) ||
            (!pair && (st = qk::launch_silu_mul_quantize(m->gate, m->up, m->xq, m->xscale, c.hidden, s))) ||
            (st = qk::launch_gemv_i8(&down, 1, m->xq, c.hidden, m->xscale, c.hidden / 32, c.hidden, 1, nullptr, 1, s)) ||
            (st = trace_copy(m->trace_x ? m->trace_x + static_cast<size_t>(l) * dim : nullptr, m->x,
                             dim * sizeof(float), s)))
            return st;
    }
    for (int l = 0; l < c.layers && !staged; ++l) {
        const qk_llama_layer &L = m->layers[l];
        if ((st = norm_quant(L.attn_norm)) || (st = trace_q(l, 0, dim))) return st;
        const qk_matrix qkv[3] = {{L.q_type, dim, L.q, m->q}, {L.k_type, kv, L.k, m->k}, {L.v_type, kv, L.v, m->v}};
        if ((st = gemv_by_mode(m, qkv, 3, m->xn, dim, s))) return st;
        attn.layer = l;
        if ((st = qk::launch_split_attention(attn, 0, m->attn_ws, m->attn_ws_bytes, s))) return st;
        if (int8_type(m, L.o_type) &&
            ((st = qk_quantize_x32(m->attn, dim, m->xq, dim, m->xscale, dim / 32, dim, 1, s)) ||
             (st = trace_q(l, 1, dim))))
            return st;
        if ((st = residual_by_mode(m, L.o_type, dim, L.o, m->attn, dim, s))) return st;
        if ((st = norm_quant(L.ffn_norm)) || (st = trace_q(l, 2, dim))) return st;
        const qk_matrix gu[2] = {{L.gate_type, c.hidden, L.gate, m->gate}, {L.up_type, c.hidden, L.up, m->up}};
        if ((st = gemv_by_mode(m, gu, 2, m->xn, dim, s))) return st;
        if (int8_type(m, L.down_type))
            st = qk::launch_silu_mul_quantize(m->gate, m->up, m->xq, m->xscale, c.hidden, s);
        else
            st = qk_silu_mul_f32(m->gate, m->up, c.hidden, s);
        if (st || (int8_type(m, L.down_type) && (st = trace_q(l, 3, c.hidden))) ||
            (st = residual_by_mode(m, L.down_type, dim, L.down, m->gate, c.hidden, s)) ||
            (st = trace_copy(m->trace_x ? m->trace_x + static_cast<size_t>(l) * dim : nullptr, m->x,
                             dim * sizeof(float), s)))
            return st;
    }
    if (!need_logits) return QK_OK;
    const void *out_w = m->w.output ? m->w.output : m->w.token_embd;
    const int out_type = m->w.output ? m->w.output_type : m->w.embd_type;
    const qk_matrix head{out_type, c.vocab, out_w, m->logits};
    if (int8_type(m, out_type)) {
        // The greedy pick in the LM head's epilogue (one pass fewer); in the
        // staged step the LM head also normalises and quantizes its input.
        float *arg_v = static_cast<float *>(m->argmax_ws);
        int *arg_i = reinterpret_cast<int *>(arg_v + qk::kArgPartsMax);
        int parts = 0;
        if (staged) {
            if ((st = qk::launch_gemv_i8_staged_argmax(&head, m->x, m->w.output_norm, c.eps, dim, arg_v, arg_i, &parts,
                                                       s)))
                return st;
        } else if ((st = norm_quant(m->w.output_norm)) ||
                   (st = qk::launch_gemv_i8_argmax(&head, m->xq, m->xscale, dim, arg_v, arg_i, &parts, s))) {
            return st;
        }
        m->next_mirrored = true;
        qk::NextEmbedding ne;
        ne.table = static_cast<const uint8_t *>(m->w.token_embd);
        ne.type = m->w.embd_type;
        ne.nb = dim / 256;
        ne.row_bytes = qk::row_bytes(m->w.embd_type, dim / 256);
        ne.out = m->x_next;
        if ((st = qk::launch_argmax_final(arg_v, arg_i, parts, m->d_next, s, m->hd_next, &ne))) return st;
        m->x_next_valid = true;
        return QK_OK;
    }
    if ((st = norm_quant(m->w.output_norm))) return st;
    if ((st = gemv_by_mode(m, &head, 1, m->xn, dim, s))) return st;
    return qk_argmax_f32(m->logits, c.vocab, m->d_next, m->argmax_ws, s);
}

// Whether the FP32 step can run over activation records: every GEMV shape
// has a record launch plan, gate and up share a type, and head_dim splits
// into whole 16-value records.
bool records_supported(const qk_llama_config &c, const std::vector<qk_llama_layer> &layers, int head_dim) {
    if (head_dim % 16 || !qk::rec_gemv_supported(c.dim, false) || !qk::rec_gemv_supported(c.dim, true) ||
        !qk::rec_gemv_supported(c.hidden, false))
        return false;
    for (const qk_llama_layer &L : layers) {
        const qk_matrix qkv[3] = {{L.q_type, c.dim, L.q, nullptr}, {L.k_type, 1, L.k, nullptr},
                                  {L.v_type, 1, L.v, nullptr}};
        const qk_matrix gu[2] = {{L.gate_type, c.hidden, L.gate, nullptr}, {L.up_type, c.hidden, L.up, nullptr}};
        const qk_matrix o{L.o_type, c.dim, L.o, nullptr}, down{L.down_type, c.dim, L.down, nullptr};
        if (!qk::rec_gemv_types(qkv, 3, false) || !qk::rec_gemv_types(gu, 2, true) ||
            !qk::rec_gemv_types(&o, 1, false) || !qk::rec_gemv_types(&down, 1, false))
            return false;
    }
    return true;
}

// The FP32 step over activation records, in five launches per layer with
// no activation staging inside any GEMV: QKV (RMSNorm as an output scale),
// attention (RoPE + KV write, records of its output), o (+ residual,
// records of x * ffn_norm), gate/up (records of SiLU(gate) * up), down
// (+ residual, records of x * the next RMSNorm's gain); then the LM head
// with its greedy pick.
int forward_records(qk_llama *m, const int32_t *tok, int pos, bool need_logits, hipStream_t s) {
    const qk_llama_config &c = m->cfg;
    const int dim = c.dim, kv = m->kv_dim;
    int st;
    if ((st = qk::launch_embedding_records(m->w.embd_type, m->w.token_embd, tok, dim, c.vocab, m->x,
                                           m->layers[0].attn_norm, m->rec_norm, m->ss_norm, s)))
        return st;
    qk::SplitAttention attn{};
    attn.q = m->q;
    attn.k = m->k;
    attn.v = m->v;
    attn.cosine = m->cosine;
    attn.sine = m->sine;
    attn.key_cache = m->key_cache;
    attn.head_major = 1;
    attn.value_cache = m->value_cache;
    attn.out = m->attn;
    attn.rec_out = m->rec_attn;
    attn.cache_rows = c.context;
    attn.rows_hint = pos + 1;
    attn.pos = attn.max_pos = pos;
    // The attention's rows split into rounds of 128 per workgroup (at most
    // 8 splits), merged by the o GEMV, which makes the records itself.
    const bool merge_o = c.heads * m->head_dim == dim && qk::rec_gemv_mergeable(dim, m->head_dim);
    attn.wide_split_rows = merge_o ? decode_split_rows(pos + 1) : 0;
    attn.defer_merge = merge_o;
    attn.n_tokens = 1;
    attn.heads = c.heads;
    attn.kv_heads = c.kv_heads;
    attn.head_dim = m->head_dim;
    qk::RecGemv qkv_in, o_out, gu_io, down_out;
    qkv_in.rec = m->rec_norm;
    qkv_in.ss = m->ss_norm;
    qkv_in.norm_eps = c.eps;
    o_out.rec = m->rec_attn;
    o_out.accumulate = 1;
    o_out.rec_out = m->rec_ffn;
    o_out.ss_out = m->ss_ffn;
    gu_io.rec = m->rec_ffn;
    gu_io.ss = m->ss_ffn;
    gu_io.norm_eps = c.eps;
    gu_io.pair = 1;
    gu_io.rec_out = m->rec_silu;
    down_out.rec = m->rec_silu;
    down_out.accumulate = 1;
    down_out.rec_out = m->rec_norm;
    down_out.ss_out = m->ss_norm;
    for (int l = 0; l < c.layers; ++l) {
        const qk_llama_layer &L = m->layers[l];
        const qk_matrix qkv[3] = {{L.q_type, dim, L.q, m->q}, {L.k_type, kv, L.k, m->k}, {L.v_type, kv, L.v, m->v}};
        if ((st = qk::launch_rec_gemv(qkv, 3, dim, qkv_in, s))) return st;
        attn.layer = l;
        int parts = 1;
        if ((st = qk::launch_split_attention(attn, 0, m->attn_ws, m->attn_ws_bytes, s, &parts))) return st;
        const qk_matrix o{L.o_type, dim, L.o, m->x};
        o_out.gain = L.ffn_norm;
        o_out.parts = parts > 1 ? static_cast<const float *>(m->attn_ws) : nullptr;
        o_out.n_parts = parts;
        o_out.part_hd = m->head_dim;
        if ((st = qk::launch_rec_gemv(&o, 1, dim, o_out, s))) return st;
        const qk_matrix gu[2] = {{L.gate_type, c.hidden, L.gate, m->gate}, {L.up_type, c.hidden, L.up, m->up}};
        if ((st = qk::launch_rec_gemv(gu, 2, dim, gu_io, s))) return st;
        const qk_matrix down{L.down_type, dim, L.down, m->x};
        down_out.gain = l + 1 < c.layers ? m->layers[l + 1].attn_norm : m->w.output_norm;
        if ((st = qk::launch_rec_gemv(&down, 1, c.hidden, down_out, s)) ||
            (st = trace_copy(m->trace_x ? m->trace_x + static_cast<size_t>(l) * dim : nullptr, m->x,
                             dim * sizeof(float), s)))
            return st;
    }
    if (!need_logits) return QK_OK;
    qk::RecGemv head_in;
    head_in.rec = m->rec_norm;
    head_in.ss = m->ss_norm;
    head_in.norm_eps = c.eps;
    head_in.arg_v = static_cast<float *>(m->argmax_ws);
    head_in.arg_i = reinterpret_cast<int *>(head_in.arg_v + qk::kArgPartsMax);
    int parts = 0;
    head_in.arg_parts = &parts;
    const void *out_w = m->w.output ? m->w.output : m->w.token_embd;
    const int out_type = m->w.output ? m->w.output_type : m->w.embd_type;
    const qk_matrix head{out_type, c.vocab, out_w, m->logits};
    if ((st = qk::launch_rec_gemv(&head, 1, dim, head_in, s))) return st;
    m->next_mirrored = true;
    return qk::launch_argmax_final(head_in.arg_v, head_in.arg_i, parts, m->d_next, s, m->hd_next);
}

}  // namespace

extern "C" {

int qk_llama_set_int8(qk_llama *m, int q4k_int8, int q6k_int8) {
    if (!m) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_set_int8: null handle");
    m->int8_q4k = q4k_int8 != 0;
    m->int8_q6k = q6k_int8 != 0;
    return qk::ok();
}

int qk_llama_create(const qk_llama_config *cfg, const qk_llama_weights *w, qk_stream stream, qk_llama **out) {
    if (!cfg || !w || !out || !w->layers || !w->token_embd || !w->output_norm)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_create: null argument");
    const qk_llama_config &c = *cfg;
    if (c.dim < 256 || c.dim % 256 || c.hidden % 256 || c.hidden < 256 || c.layers < 1 || c.heads < 1 ||
        c.kv_heads < 1 || c.dim % c.heads || c.heads % c.kv_heads || c.vocab < 1 || c.context < 1)
        return qk::fail(QK_ERR_SHAPE, "qk_llama_create: unsupported model shape");
    const int head_dim = c.dim / c.heads;
    if (!qk::gemv_fusable(c.dim) || !qk::gemv_fusable(c.hidden))
        return qk::fail(QK_ERR_LIMIT, "qk_llama_create: dim or hidden too long to stage the activations of a step");
    if (!qk::aligned(w->output_norm, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_llama_create: norm weights must be 16-byte aligned");
    for (int l = 0; l < c.layers; ++l)
        if (!qk::aligned(w->layers[l].attn_norm, 16) || !qk::aligned(w->layers[l].ffn_norm, 16))
            return qk::fail(QK_ERR_ALIGN, "qk_llama_create: norm weights must be 16-byte aligned");
    if (head_dim % 4 || 256 % head_dim)
        return qk::fail(QK_ERR_LIMIT, "qk_llama_create: head_dim must be a multiple of 4 dividing 256");
    if (!quant_type(w->embd_type) || (w->output && !quant_type(w->output_type)))
        return qk::fail(QK_ERR_TYPE, "qk_llama_create: embedding and output must be Q4_K or Q6_K (either layout)");
    for (int l = 0; l < c.layers; ++l) {
        const qk_llama_layer &L = w->layers[l];
        if (!quant_type(L.q_type) || !quant_type(L.k_type) || !quant_type(L.v_type) || !quant_type(L.o_type) ||
            !quant_type(L.gate_type) || !quant_type(L.up_type) || !quant_type(L.down_type))
            return qk::fail(QK_ERR_TYPE, "qk_llama_create: layer " + std::to_string(l) + " has a non-K-quant tensor");
        if (!L.q || !L.k || !L.v || !L.o || !L.gate || !L.up || !L.down || !L.attn_norm || !L.ffn_norm)
            return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_create: layer " + std::to_string(l) + " is incomplete");
    }
    if (!qk::attention_supported(c.heads / c.kv_heads, head_dim))
        return qk::fail(QK_ERR_LIMIT, "qk_llama_create: head layout outside the attention kernel");

    qk_llama *m = new qk_llama();
    m->cfg = c;
    m->w = *w;
    m->layers.assign(w->layers, w->layers + c.layers);
    m->w.layers = m->layers.data();
    m->stream = static_cast<hipStream_t>(stream);
    m->head_dim = head_dim;
    m->kv_dim = head_dim * c.kv_heads;
    const size_t cache = static_cast<size_t>(c.layers) * c.context * m->kv_dim;
    const int half = head_dim / 2;
    m->attn_ws_bytes = qk::split_attention_workspace_bytes(1, c.heads, c.kv_heads, head_dim, c.context);
    // Everything create allocates: caches, split Q6_K copies, activation
    // buffers, RoPE tables, workspaces and the activation records.
    const size_t argmax_bytes = std::max(2 * qk::kArgPartsMax * sizeof(float), qk_argmax_workspace_bytes(c.vocab));
    const uint64_t buffer_bytes =
        sizeof(float) * (5ull * c.dim + 2ull * m->kv_dim + 2ull * c.hidden + c.vocab + 2ull * c.context * half) +
        argmax_bytes + 2 * sizeof(int32_t) + std::max(c.dim, c.hidden) / 32 * (32 + sizeof(float)) + m->attn_ws_bytes +
        (4ull * c.dim / 16 + c.hidden / 16) * sizeof(qk::XGroup) + 2ull * c.dim / 16 * sizeof(float);
    int st = check_free_memory("qk_llama_create",
                               2 * cache * sizeof(float) + split_copy_bytes(*w, c, m->kv_dim) + buffer_bytes);
    if (st) {
        delete m;
        return st;
    }
    if ((st = dev_alloc(m->mem.buffers, &m->x, c.dim, "residual")) ||
        (st = dev_alloc(m->mem.buffers, &m->x_next, c.dim, "next embedding")) ||
        (st = dev_alloc(m->mem.buffers, &m->xn, c.dim, "normalized state")) ||
        (st = dev_alloc(m->mem.buffers, &m->q, c.dim, "query")) || (st = dev_alloc(m->mem.buffers, &m->k, m->kv_dim, "key")) ||
        (st = dev_alloc(m->mem.buffers, &m->v, m->kv_dim, "value")) || (st = dev_alloc(m->mem.buffers, &m->attn, c.dim, "attention")) ||
        (st = dev_alloc(m->mem.buffers, &m->tmp, c.dim, "residual update")) || (st = dev_alloc(m->mem.buffers, &m->gate, c.hidden, "gate")) ||
        (st = dev_alloc(m->mem.buffers, &m->up, c.hidden, "up projection")) || (st = dev_alloc(m->mem.buffers, &m->logits, c.vocab, "logits")) ||
        (st = dev_alloc(m->mem.kv_cache, &m->key_cache, cache, "key cache")) ||
        (st = dev_alloc(m->mem.kv_cache, &m->value_cache, cache, "value cache")) ||
        (st = dev_alloc(m->mem.buffers, &m->cosine, static_cast<size_t>(c.context) * half, "RoPE cosine")) ||
        (st = dev_alloc(m->mem.buffers, &m->sine, static_cast<size_t>(c.context) * half, "RoPE sine")) ||
        // The FP32 step's LM-head partials, or the INT8 step's qk_argmax_f32
        // workspace, whichever is larger (the latter grows with vocab).
        (st = dev_alloc(m->mem.buffers, reinterpret_cast<uint8_t **>(&m->argmax_ws), argmax_bytes,
                        "argmax partials")) ||
        (st = dev_alloc(m->mem.buffers, &m->d_next, 1, "next token")) || (st = dev_alloc(m->mem.buffers, &m->d_token, 1, "input token")) ||
        (st = dev_alloc(m->mem.buffers, &m->xq, std::max(c.dim, c.hidden), "quantized activations")) ||
        (st = dev_alloc(m->mem.buffers, &m->xscale, std::max(c.dim, c.hidden) / 32, "activation scales"))) {
        release(m);
        return st;
    }
    if (m->attn_ws_bytes &&
        (st = dev_alloc(m->mem.buffers, reinterpret_cast<uint8_t **>(&m->attn_ws), m->attn_ws_bytes, "attention workspace"))) {
        release(m);
        return st;
    }
    if (hipHostMalloc(reinterpret_cast<void **>(&m->h_token), 2 * sizeof(int32_t), hipHostMallocDefault) !=
            hipSuccess ||
        hipHostMalloc(reinterpret_cast<void **>(&m->h_next), sizeof(int32_t),
                      hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void **>(&m->hd_next), m->h_next, 0) != hipSuccess ||
        hipEventCreateWithFlags(&m->upload_done, hipEventDisableTiming) != hipSuccess) {
        release(m);
        return qk::fail(QK_ERR_DEVICE, "qk_llama_create: cannot allocate pinned staging");
    }
    // RoPE tables exactly as the reference builds them on the host
    // (inferencer.cu:1218-1226): float powf, float angle, cosf / sinf.
    std::vector<float> cosines(static_cast<size_t>(c.context) * half), sines(cosines.size()), freq(half);
    for (int i = 0; i < half; ++i) freq[i] = std::pow(c.rope_theta, -2.f * static_cast<float>(i) / head_dim);
    for (int pos = 0; pos < c.context; ++pos)
        for (int i = 0; i < half; ++i) {
            const float angle = static_cast<float>(pos) * freq[i];
            cosines[static_cast<size_t>(pos) * half + i] = std::cos(angle);
            sines[static_cast<size_t>(pos) * half + i] = std::sin(angle);
        }
    if (hipMemcpy(m->cosine, cosines.data(), cosines.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->sine, sines.data(), sines.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(m->key_cache, 0, cache * sizeof(float)) != hipSuccess ||
        hipMemset(m->value_cache, 0, cache * sizeof(float)) != hipSuccess) {
        release(m);
        return qk::fail(QK_ERR_DEVICE, "qk_llama_create: table upload failed");
    }
    if ((st = split_weights(m->owned, m->mem.weight_copies, m->w, m->layers, c, m->kv_dim, m->stream))) {
        release(m);
        return st;
    }
    m->w.layers = m->layers.data();
    const int head_type = m->w.output ? m->w.output_type : m->w.embd_type;
    const qk_matrix head{head_type, c.vocab, m->w.output ? m->w.output : m->w.token_embd, nullptr};
    m->records = records_supported(c, m->layers, head_dim) && qk::rec_gemv_types(&head, 1, false);
    if (m->records) {
        const size_t gd = static_cast<size_t>(c.dim) / 16, gh = static_cast<size_t>(c.hidden) / 16;
        if ((st = dev_alloc(m->mem.buffers, &m->rec_norm, gd, "activation records")) ||
            (st = dev_alloc(m->mem.buffers, &m->rec_attn, gd, "activation records")) ||
            (st = dev_alloc(m->mem.buffers, &m->rec_ffn, gd, "activation records")) ||
            (st = dev_alloc(m->mem.buffers, &m->rec_silu, gh, "activation records")) ||
            (st = dev_alloc(m->mem.buffers, &m->ss_norm, gd, "record sums of squares")) ||
            (st = dev_alloc(m->mem.buffers, &m->ss_ffn, gd, "record sums of squares"))) {
            release(m);
            return st;
        }
    }
    *out = m;
    return qk::ok();
}

int qk_llama_destroy(qk_llama *m) {
    if (!m) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_destroy: null handle");
    (void)hipStreamSynchronize(m->stream);
    release(m);
    return qk::ok();
}

int qk_llama_kv_cache(qk_llama *m, float **key_cache, float **value_cache) {
    if (!m || !key_cache || !value_cache) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_kv_cache: null argument");
    *key_cache = m->key_cache;
    *value_cache = m->value_cache;
    return qk::ok();
}

int qk_llama_memory_bytes(const qk_llama *m, qk_llama_memory *out) {
    if (!m || !out) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_memory_bytes: null argument");
    *out = m->mem;
    return qk::ok();
}

int qk_llama_logits(qk_llama *m, const float **logits) {
    if (!m || !logits) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_logits: null argument");
    *logits = m->logits;
    return qk::ok();
}

int qk_llama_set_trace(qk_llama *m, float *residuals, int8_t *quantized) {
    if (!m) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_set_trace: null handle");
    if ((residuals && !qk::aligned(residuals, 4)))
        return qk::fail(QK_ERR_ALIGN, "qk_llama_set_trace: residuals must be 4-byte aligned");
    m->trace_x = residuals;
    m->trace_q = quantized;
    return qk::ok();
}

int qk_llama_matrix_calls(const qk_llama *m, uint64_t *calls) {
    if (!m || !calls) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_matrix_calls: null argument");
    *calls = m->matrix_calls;
    return qk::ok();
}

int qk_llama_residual(qk_llama *m, const float **x) {
    if (!m || !x) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_residual: null argument");
    *x = m->x;
    return qk::ok();
}

int qk_llama_forward(qk_llama *m, int token, int pos, int need_logits, int *next_token) {
    if (!m) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_forward: null handle");
    const qk_llama_config &c = m->cfg;
    if (pos < 0 || pos >= c.context || token < 0 || token >= c.vocab)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_forward: token or position outside model context");
    hipStream_t s = m->stream;
    const int dim = c.dim, kv = m->kv_dim, hd = m->head_dim;
    int st;
    const int32_t *tok = m->d_next;
    const bool embedded = token == m->last_next && m->x_next_valid;
    m->x_next_valid = false;
    if (token != m->last_next) {
        // A step without logits returns before its work runs: the pinned slot
        // is rewritten only once the previous upload has read it.
        if (m->upload_pending && hipEventSynchronize(m->upload_done) != hipSuccess)
            return qk::fail(QK_ERR_DEVICE, "qk_llama_forward: stream error");
        m->h_token[0] = token;
        if (hipMemcpyAsync(m->d_token, m->h_token, sizeof(int32_t), hipMemcpyHostToDevice, s) != hipSuccess ||
            hipEventRecord(m->upload_done, s) != hipSuccess)
            return qk::fail(QK_ERR_DEVICE, "qk_llama_forward: token upload failed");
        m->upload_pending = true;
        tok = m->d_token;
    }
    m->last_next = -1;
    m->next_mirrored = false;
    // Seven matrix products per layer (q, k, v, o, gate, up, down) and the
    // LM head, counted as the reference counts FastGPU::matvec and its fused
    // qkv / gate-up launches (inferencer.cu:1170, 1457, 1500).
    m->matrix_calls += 7ull * c.layers + (need_logits ? 1 : 0);
    if (m->int8_q4k || m->int8_q6k) {
        if ((st = forward_int8(m, tok, pos, need_logits != 0, embedded, s))) return st;
        if (!need_logits) {
            if (next_token) *next_token = -1;
            return qk::ok();
        }
    } else if (m->records) {
        if ((st = forward_records(m, tok, pos, need_logits != 0, s))) return st;
        if (!need_logits) {
            if (next_token) *next_token = -1;
            return qk::ok();
        }
    } else {
        if ((st = qk_embedding(m->w.embd_type, m->w.token_embd, tok, 1, m->x, dim, c.vocab, s))) return st;
        // Five launches per layer: RMSNorm is staged inside the QKV / gate-up
        // GEMVs, SiLU * up inside the down GEMV, the residual adds are their
        // epilogues, and RoPE + the KV write open the attention kernel.
        qk::GemvFusion attn_in, ffn_in, residual, down_in;
        attn_in.norm_eps = ffn_in.norm_eps = c.eps;
        residual.accumulate = down_in.accumulate = 1;
        down_in.up = m->up;
        qk::SplitAttention attn{};
        attn.q = m->q;
        attn.k = m->k;
        attn.v = m->v;
        attn.cosine = m->cosine;
        attn.sine = m->sine;
        attn.key_cache = m->key_cache;
    attn.head_major = 1;
        attn.value_cache = m->value_cache;
        attn.out = m->attn;
        attn.cache_rows = c.context;
        attn.rows_hint = pos + 1;
        attn.pos = attn.max_pos = pos;
        attn.n_tokens = 1;
        attn.heads = c.heads;
        attn.kv_heads = c.kv_heads;
        attn.head_dim = hd;
        for (int l = 0; l < c.layers; ++l) {
            const qk_llama_layer &L = m->layers[l];
            attn_in.norm_w = L.attn_norm;
            ffn_in.norm_w = L.ffn_norm;
            const qk_matrix qkv[3] = {{L.q_type, dim, L.q, m->q}, {L.k_type, kv, L.k, m->k}, {L.v_type, kv, L.v, m->v}};
            if ((st = qk::launch_gemv_fused(qkv, 3, m->x, dim, dim, 1, nullptr, attn_in, s))) return st;
            attn.layer = l;
            if ((st = qk::launch_split_attention(attn, 0, m->attn_ws, m->attn_ws_bytes, s))) return st;
            const qk_matrix o{L.o_type, dim, L.o, m->x};
            if ((st = qk::launch_gemv_fused(&o, 1, m->attn, dim, dim, 1, nullptr, residual, s))) return st;
            const qk_matrix gu[2] = {{L.gate_type, c.hidden, L.gate, m->gate}, {L.up_type, c.hidden, L.up, m->up}};
            if ((st = qk::launch_gemv_fused(gu, 2, m->x, dim, dim, 1, nullptr, ffn_in, s))) return st;
            const qk_matrix down{L.down_type, dim, L.down, m->x};
            if ((st = qk::launch_gemv_fused(&down, 1, m->gate, c.hidden, c.hidden, 1, nullptr, down_in, s)) ||
                (st = trace_copy(m->trace_x ? m->trace_x + static_cast<size_t>(l) * dim : nullptr, m->x,
                                 dim * sizeof(float), s)))
                return st;
        }
        if (!need_logits) {
            if (next_token) *next_token = -1;
            return qk::ok();
        }
        // The LM head's epilogue keeps each workgroup's best logit (argmax_blocks_cuda
        // folded in); one small kernel picks the token from those partials.
        qk::GemvFusion out_in;
        out_in.norm_w = m->w.output_norm;
        out_in.norm_eps = c.eps;
        out_in.arg_v = static_cast<float *>(m->argmax_ws);
        out_in.arg_i = reinterpret_cast<int *>(out_in.arg_v + qk::kArgPartsMax);
        int parts = 0;
        out_in.arg_parts = &parts;
        const void *out_w = m->w.output ? m->w.output : m->w.token_embd;
        const int out_type = m->w.output ? m->w.output_type : m->w.embd_type;
        const qk_matrix head{out_type, c.vocab, out_w, m->logits};
        if ((st = qk::launch_gemv_fused(&head, 1, m->x, dim, dim, 1, nullptr, out_in, s))) return st;
        m->next_mirrored = true;
        if ((st = qk::launch_argmax_final(out_in.arg_v, out_in.arg_i, parts, m->d_next, s, m->hd_next))) return st;
    }
    if (m->next_mirrored) {
        if (hipStreamSynchronize(s) != hipSuccess)
            return qk::fail(QK_ERR_DEVICE, "qk_llama_forward: next token wait failed");
        m->last_next = *static_cast<volatile int32_t *>(m->h_next);
    } else {
        if (hipMemcpyAsync(m->h_token + 1, m->d_next, sizeof(int32_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return qk::fail(QK_ERR_DEVICE, "qk_llama_forward: next token download failed");
        m->last_next = m->h_token[1];
    }
    m->upload_pending = false;   // the synchronisation retired every upload
    if (next_token) *next_token = m->last_next;
    return qk::ok();
}

}  // extern "C"

// ------------------------------------------------------- ragged batches --

struct qk_llama_batch {
    qk_llama_config cfg{};
    qk_llama_weights w{};
    std::vector<qk_llama_layer> layers;
    hipStream_t stream = nullptr;
    int head_dim = 0, kv_dim = 0, max_tokens = 0;
    int64_t cache_rows = 0;
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *tmp = nullptr;
    float *gate = nullptr, *up = nullptr, *logits = nullptr;
    float *key_cache = nullptr, *value_cache = nullptr, *cosine = nullptr, *sine = nullptr;
    void *gemm_ws = nullptr, *argmax_ws = nullptr, *attn_ws = nullptr;
    size_t gemm_ws_bytes = 0, attn_ws_bytes = 0;
    // Matrix-core steps (8 tokens and more) run as a chain: each projection's
    // reduction packs the next one's input records (rec_a: o -> gate/up and
    // down -> next QKV, with the RMSNorm deferred through ss; rec_b: gate/up
    // -> down).
    uint8_t *rec_a = nullptr, *rec_b = nullptr;
    float *ss = nullptr;
    int32_t *d_tokens = nullptr, *d_next = nullptr, *d_rows = nullptr;
    qk_batch_token *d_desc = nullptr;
    uint8_t *h_stage = nullptr;   // pinned: tokens, descriptors, logit rows, results
    std::vector<void *> owned;    // split-layout copies of the Q6_K weights
    std::vector<int64_t> kv_writes;   // host scratch of the KV-row check
    qk_llama_memory mem{};        // device bytes the handle holds
    uint64_t matrix_calls = 0;    // quantized matrix products issued (FastGPU::calls)
    // INT8 mode (qk_llama_batch_set_int8; buffers made at its first enable):
    // quantized inputs of dim (xq / xs) and hidden (hq / hs) columns per
    // token, and the split sums of the matrix-core products.
    int int8 = 0;
    int8_t *xq = nullptr, *hq = nullptr;
    float *xs = nullptr, *hs = nullptr;
    void *i8_ws = nullptr;
    size_t i8_ws_bytes = 0;
    // The LM head in GGUF blocks (a Q6_K head only; made from the split
    // copy at the first enable): the multi-token INT8 product walks row tiles
    // block by block, and in the split layout each block of a 32-row tile
    // touches parts of ~6 cache lines per row -- about 6 MB of lines per
    // step on an XCD, more than its 4 MB L2, so each line was fetched twice
    // (FETCH 2.0x the matrix, 84.5 us at 32 tokens); in 210-byte blocks it is
    // 1.11x and 77.9 us.
    uint8_t *head_q6k = nullptr;
    // qk_llama_batch_set_trace: per token the residual after each layer
    // [token][layer][dim] and the INT8 inputs of each layer's products
    // [token][layer][4][max(dim, hidden)].
    float *trace_x = nullptr;
    int8_t *trace_q = nullptr;
};

namespace {

void release_batch(qk_llama_batch *m) {
    void *bufs[] = {m->x, m->xn, m->q, m->k, m->v, m->attn, m->tmp, m->gate, m->up, m->logits, m->key_cache,
                    m->value_cache, m->cosine, m->sine, m->gemm_ws, m->argmax_ws, m->attn_ws, m->d_tokens, m->d_next,
                    m->d_rows, m->d_desc, m->rec_a, m->rec_b, m->ss, m->xq, m->hq, m->xs, m->hs, m->i8_ws,
                    m->head_q6k};
    for (void *b : bufs)
        if (b) (void)hipFree(b);
    if (m->h_stage) (void)hipHostFree(m->h_stage);
    for (void *b : m->owned) (void)hipFree(b);
    delete m;
}

// Pinned staging of one step: tokens, next tokens and logit rows (int32 each),
// then the descriptors.
size_t stage_bytes(int max_tokens) {
    return static_cast<size_t>(max_tokens) * (3 * sizeof(int32_t) + sizeof(qk_batch_token));
}

// The KV rows a step writes are kv_row + pos, one per token.  Two tokens
// writing one row race, so that is an error.  A token reads rows kv_row ..
// kv_row + pos; when some of those are written by other tokens of the same
// step (several tokens of one sequence: a prefill chunk), every row must be
// written before attention reads any (*chained).  Descriptors are already
// range-checked, so kv_row + pos does not overflow.
int check_kv_rows(const qk_batch_token *desc, int n, std::vector<int64_t> &writes, bool *chained) {
    writes.resize(n);
    for (int t = 0; t < n; ++t) writes[t] = desc[t].kv_row + desc[t].pos;
    std::sort(writes.begin(), writes.end());
    for (int t = 1; t < n; ++t)
        if (writes[t] == writes[t - 1])
            return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: two tokens write KV row " +
                                                    std::to_string(writes[t]) + " (same sequence and position)");
    *chained = false;
    for (int t = 0; t < n && !*chained; ++t) {
        const auto lo = std::lower_bound(writes.begin(), writes.end(), desc[t].kv_row);
        const auto hi = std::lower_bound(writes.begin(), writes.end(), desc[t].kv_row + desc[t].pos);
        *chained = lo != hi;   // another token writes a row this one reads
    }
    return QK_OK;
}

// The residual of the step's T tokens after layer l into the trace.
int batch_trace_x(qk_llama_batch *m, int l, int T, hipStream_t s) {
    const size_t row = static_cast<size_t>(m->cfg.dim) * sizeof(float);
    return trace_copy_2d(m->trace_x ? m->trace_x + static_cast<size_t>(l) * m->cfg.dim : nullptr, m->cfg.layers * row,
                         m->x, row, row, T, s);
}

// INT8 products of T tokens (the reference's dp4a paths): the GEMV kernels
// below 8 tokens, the integer matrix cores from 8 on.
int batch_gemm_i8(qk_llama_batch *m, const qk_matrix *mats, int n, const int8_t *xq, const float *xs, int cols, int T,
                  bool accumulate, hipStream_t s) {
    int ldy[QK_MAX_FUSED];
    for (int i = 0; i < n; ++i) ldy[i] = mats[i].rows;
    if (T < 8) return qk::launch_gemv_i8(mats, n, xq, cols, xs, cols / 32, cols, T, ldy, accumulate, s);
    return qk::launch_skinny_i8(mats, n, ldy, xq, cols, xs, cols / 32, cols, T, accumulate, nullptr, nullptr, 0, 0,
                                m->i8_ws, m->i8_ws_bytes, s, "qk_llama_batch_forward");
}

// The layers of an INT8 step, the reference's batched INT8 arithmetic
// (FastRunner::prefill, inferencer.cu:1279-1423) for any ragged batch: per
// layer RMSNorm and quantization of x (rmsnorm_quantize_batch_cuda), the
// fused QKV product (qkv_batch_cuda), RoPE + KV write + attention, the
// attention output quantized and o added into x (batch_matvec +
// add_batch_cuda), RMSNorm and quantization, gate / up with SiLU(gate) * up
// quantized (gate_up_batch_cuda, silu_batch_cuda, and down's quantization),
// down added into x.
int batch_layers_int8(qk_llama_batch *m, int T, bool chained, qk::SplitAttention &attn, hipStream_t s,
                      const float *head_norm, bool *head_normed) {
    const qk_llama_config &c = m->cfg;
    const int dim = c.dim, hidden = c.hidden, kv = m->kv_dim, hd = m->head_dim;
    int st;
    auto norm_quant = [&](const float *w) {
        return qk_rmsnorm_quantize_x32(m->x, dim, w, nullptr, 0, m->xq, dim, m->xs, dim / 32, dim, T, c.eps, s);
    };
    const size_t qstride = std::max(dim, hidden);
    auto trace_q = [&](int l, int stage, const int8_t *src, int cols) {
        return trace_copy_2d(m->trace_q ? m->trace_q + (l * 4 + stage) * qstride : nullptr, c.layers * 4 * qstride,
                             src, cols, cols, T, s);
    };
    // down's split reduction normalises and quantizes the next layer's
    // input itself when it can (qk::SkNorm; the same codes): normed says it
    // did.  A step tracing its INT8 inputs plans the same launch and keeps
    // the separate normalisation.
    int normed = 0;
    for (int l = 0; l < c.layers; ++l) {
        const qk_llama_layer &L = m->layers[l];
        const qk_matrix qkv[3] = {{L.q_type, dim, L.q, m->q}, {L.k_type, kv, L.k, m->k}, {L.v_type, kv, L.v, m->v}};
        // A decode batch's attention reads q, k and v once, so it adds the
        // QKV product's split sums itself (no reduction launch; the product
        // then splits its rows over twice the workgroups).
        qk::SkDeferred qd;
        if ((!normed && (st = norm_quant(L.attn_norm))) || (st = trace_q(l, 0, m->xq, dim)))
            return st;
        if (T >= 8 && !chained) {
            const int ldy[3] = {dim, kv, kv};
            if ((st = qk::launch_skinny_i8(qkv, 3, ldy, m->xq, dim, m->xs, dim / 32, dim, T, 0, nullptr, nullptr, 0, 0,
                                           m->i8_ws, m->i8_ws_bytes, s, "qk_llama_batch_forward", nullptr, &qd)))
                return st;
        } else if ((st = batch_gemm_i8(m, qkv, 3, m->xq, m->xs, dim, T, false, s))) {
            return st;
        }
        attn.qkv_parts = qd.partials;
        attn.qkv_splits = qd.splits;
        attn.qkv_ttiles = qd.token_tiles;
        for (int i = 0; i < 3; ++i) attn.qkv_tile0[i] = qd.tile_begin[i];
        if (chained &&
            (st = qk::launch_rope_kv_batched(m->q, m->k, m->v, m->cosine, m->sine, m->key_cache, m->value_cache, l,
                                             m->cache_rows, m->d_desc, T, c.context, c.heads, c.kv_heads, hd, 1, s)))
            return st;
        attn.layer = l;
        attn.gemm_rec = nullptr;
        // The attention quantizes its own outputs for o (quantize_batch_cuda's
        // codes) when its rows are the o projection's input rows.
        const bool q8 = c.heads * hd == dim && hd % 32 == 0;
        attn.q8_out = q8 ? m->xq : nullptr;
        attn.q8_scale = q8 ? m->xs : nullptr;
        if ((st = qk::launch_split_attention(attn, 0, m->attn_ws, m->attn_ws_bytes, s))) return st;
        attn.q8_out = nullptr;
        attn.q8_scale = nullptr;
        attn.qkv_parts = nullptr;
        attn.qkv_splits = 0;
        const qk_matrix o{L.o_type, dim, L.o, m->x};
        // (Folding the FFN's RMSNorm into o the same way makes o split its
        // sums, which it otherwise does not: no faster, 1.650 -> 1.653-1.658
        // ms for the 32-sequence step.)
        if ((!q8 && (st = qk_quantize_x32(m->attn, dim, m->xq, dim, m->xs, dim / 32, dim, T, s))) ||
            (st = trace_q(l, 1, m->xq, dim)) || (st = batch_gemm_i8(m, &o, 1, m->xq, m->xs, dim, T, true, s)) ||
            (st = norm_quant(L.ffn_norm)) || (st = trace_q(l, 2, m->xq, dim)))
            return st;
        const qk_matrix gu[2] = {{L.gate_type, hidden, L.gate, m->gate}, {L.up_type, hidden, L.up, m->up}};
        if (T >= 8 && L.gate_type == L.up_type) {
            // SiLU(gate) * up quantized in the product's own epilogue.
            if ((st = qk::launch_skinny_i8(gu, 2, nullptr, m->xq, dim, m->xs, dim / 32, dim, T, 0, m->hq, m->hs, hidden,
                                           hidden / 32, m->i8_ws, m->i8_ws_bytes, s, "qk_llama_batch_forward")))
                return st;
        } else if ((st = batch_gemm_i8(m, gu, 2, m->xq, m->xs, dim, T, false, s)) ||
                   (st = qk::launch_silu_mul_quantize(m->gate, m->up, m->hq, m->hs, T * hidden, s))) {
            return st;
        }
        const qk_matrix down{L.down_type, dim, L.down, m->x};
        qk::SkNorm next;
        next.eps = c.eps;
        next.xq = m->xq;
        next.xs = m->xs;
        next.ldxq = dim;
        next.ldxs = dim / 32;
        next.done = &normed;
        // The last layer's reduction normalises and quantizes the LM head's
        // input (head_norm: the output norm when the head reads every token
        // in order).
        next.w = l + 1 < c.layers ? m->layers[l + 1].attn_norm : head_norm;
        next.plan_only = m->trace_q != nullptr;   // the same split sums, the separate norm
        normed = 0;
        if ((st = trace_q(l, 3, m->hq, hidden)) ||
            (st = T >= 8 && next.w
                      ? qk::launch_skinny_i8(&down, 1, nullptr, m->hq, hidden, m->hs, hidden / 32, hidden, T, 1, nullptr,
                                             nullptr, 0, 0, m->i8_ws, m->i8_ws_bytes, s, "qk_llama_batch_forward", &next)
                      : batch_gemm_i8(m, &down, 1, m->hq, m->hs, hidden, T, true, s)) ||
            (st = batch_trace_x(m, l, T, s)))
            return st;
    }
    *head_normed = head_norm && normed;
    return QK_OK;
}

}  // namespace

extern "C" {

int qk_llama_batch_set_int8(qk_llama_batch *m, int q4k_int8, int q6k_int8) {
    if (!m) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_set_int8: null handle");
    if ((q4k_int8 != 0) != (q6k_int8 != 0))
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_set_int8: the batched step runs INT8 for both Q4_K and "
                                            "Q6_K or for neither");
    if (q4k_int8 && !m->xq) {
        const qk_llama_config &c = m->cfg;
        const size_t T = static_cast<size_t>(m->max_tokens);
        const int kv = m->kv_dim;
        auto tiles = [](int rows) { return (rows + 31) / 32; };
        size_t ws = 0;
        ws = std::max(ws, qk::skinny_i8_workspace_bytes(c.dim, tiles(c.dim) + 2 * tiles(kv), m->max_tokens, false));
        ws = std::max(ws, qk::skinny_i8_workspace_bytes(c.dim, tiles(c.hidden), m->max_tokens, true));
        ws = std::max(ws, qk::skinny_i8_workspace_bytes(c.hidden, tiles(c.dim), m->max_tokens, false));
        ws = std::max(ws, qk::skinny_i8_workspace_bytes(c.dim, tiles(c.vocab), m->max_tokens, false));
        const void *head = m->w.output ? m->w.output : m->w.token_embd;
        const bool head_split = (m->w.output ? m->w.output_type : m->w.embd_type) == QK_TYPE_Q6_K_SPLIT;
        const uint64_t head_bytes = head_split ? static_cast<uint64_t>(c.vocab) * (c.dim / 256) * 210 : 0;
        const uint64_t need = T * (c.dim + c.hidden) * (1 + sizeof(float) / 32.0) + ws + head_bytes + 1024;
        int st;
        if ((st = check_free_memory("qk_llama_batch_set_int8", need))) return st;
        uint64_t bytes = 0, copies = 0;
        if ((st = dev_alloc(bytes, &m->xq, T * c.dim, "quantized activations")) ||
            (st = dev_alloc(bytes, &m->xs, T * (c.dim / 32), "activation scales")) ||
            (st = dev_alloc(bytes, &m->hq, T * c.hidden, "quantized hidden activations")) ||
            (st = dev_alloc(bytes, &m->hs, T * (c.hidden / 32), "hidden activation scales")) ||
            (ws && (st = dev_alloc(bytes, reinterpret_cast<uint8_t **>(&m->i8_ws), ws, "split sums"))) ||
            (head_bytes && (st = dev_alloc(copies, &m->head_q6k, head_bytes, "LM head in GGUF blocks"))) ||
            (head_bytes && (st = qk::launch_q6k_join(head, m->head_q6k, c.dim, c.vocab, m->stream)))) {
            for (void *b : {static_cast<void *>(m->xq), static_cast<void *>(m->xs), static_cast<void *>(m->hq),
                            static_cast<void *>(m->hs), m->i8_ws, static_cast<void *>(m->head_q6k)})
                (void)hipFree(b);
            m->xq = m->hq = nullptr;
            m->xs = m->hs = nullptr;
            m->i8_ws = nullptr;
            m->head_q6k = nullptr;
            return st;
        }
        m->i8_ws_bytes = ws;
        m->mem.buffers += bytes;
        m->mem.weight_copies += copies;
    }
    m->int8 = q4k_int8 != 0;
    return qk::ok();
}

int qk_llama_batch_create(const qk_llama_config *cfg, const qk_llama_weights *w, int max_tokens, int64_t cache_rows,
                          qk_stream stream, qk_llama_batch **out) {
    if (!cfg || !w || !out || !w->layers || !w->token_embd || !w->output_norm)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_create: null argument");
    const qk_llama_config &c = *cfg;
    if (c.dim < 256 || c.dim % 256 || c.hidden % 256 || c.hidden < 256 || c.layers < 1 || c.heads < 1 ||
        c.kv_heads < 1 || c.dim % c.heads || c.heads % c.kv_heads || c.vocab < 1 || c.context < 1)
        return qk::fail(QK_ERR_SHAPE, "qk_llama_batch_create: unsupported model shape");
    if (max_tokens < 1 || max_tokens > 4096 || cache_rows < 1)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_create: max_tokens must be 1..4096 and cache_rows >= 1");
    const int head_dim = c.dim / c.heads;
    if (!qk::attention_supported(c.heads / c.kv_heads, head_dim))
        return qk::fail(QK_ERR_LIMIT, "qk_llama_batch_create: head layout outside the attention kernel");
    if (!quant_type(w->embd_type) || (w->output && !quant_type(w->output_type)))
        return qk::fail(QK_ERR_TYPE, "qk_llama_batch_create: embedding and output must be Q4_K or Q6_K (either layout)");
    if (!qk::gemv_fusable(c.dim) || !qk::gemv_fusable(c.hidden))
        return qk::fail(QK_ERR_LIMIT, "qk_llama_batch_create: dim or hidden too long to stage the activations");
    if (!qk::aligned(w->output_norm, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_llama_batch_create: norm weights must be 16-byte aligned");
    for (int l = 0; l < c.layers; ++l)
        if (!qk::aligned(w->layers[l].attn_norm, 16) || !qk::aligned(w->layers[l].ffn_norm, 16))
            return qk::fail(QK_ERR_ALIGN, "qk_llama_batch_create: norm weights must be 16-byte aligned");
    for (int l = 0; l < c.layers; ++l) {
        const qk_llama_layer &L = w->layers[l];
        if (!quant_type(L.q_type) || !quant_type(L.k_type) || !quant_type(L.v_type) || !quant_type(L.o_type) ||
            !quant_type(L.gate_type) || !quant_type(L.up_type) || !quant_type(L.down_type))
            return qk::fail(QK_ERR_TYPE, "qk_llama_batch_create: layer " + std::to_string(l) + " has a non-K-quant tensor");
        if (!L.q || !L.k || !L.v || !L.o || !L.gate || !L.up || !L.down || !L.attn_norm || !L.ffn_norm)
            return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_create: layer " + std::to_string(l) + " is incomplete");
    }
    qk_llama_batch *m = new qk_llama_batch();
    m->cfg = c;
    m->w = *w;
    m->layers.assign(w->layers, w->layers + c.layers);
    m->w.layers = m->layers.data();
    m->stream = static_cast<hipStream_t>(stream);
    m->head_dim = head_dim;
    m->kv_dim = head_dim * c.kv_heads;
    m->max_tokens = max_tokens;
    m->cache_rows = cache_rows;
    const size_t T = static_cast<size_t>(max_tokens);
    const size_t cache = static_cast<size_t>(c.layers) * cache_rows * m->kv_dim;
    const int half = head_dim / 2;
    size_t ws = 0;
    const int kv = m->kv_dim;
    const int shapes[][2] = {{c.dim, c.dim + 2 * kv}, {c.dim, c.dim}, {c.dim, 2 * c.hidden}, {c.hidden, c.dim},
                             {c.dim, c.vocab}};
    // The workspace of a call depends on its token count through the number
    // of 32-token tiles (fewer tiles can mean more splits), so the bound is
    // taken over every tile count up to max_tokens.
    for (int tiles = 1;; ++tiles) {
        const int tq = std::min(tiles * 32, max_tokens);
        for (const auto &sh : shapes) ws = std::max(ws, qk_gemv_batched_workspace_bytes(sh[0], sh[1], tq));
        for (int i = 0; i < 4; ++i) ws = std::max(ws, qk::batched_chain_workspace_bytes(shapes[i][0], shapes[i][1], tq));
        if (tq == max_tokens) break;
    }
    m->gemm_ws_bytes = ws;
    const size_t rec_bytes = qk::batched_records_bytes(std::max(c.dim, c.hidden), max_tokens);
    m->attn_ws_bytes = qk::split_attention_workspace_bytes(max_tokens, c.heads, c.kv_heads, head_dim, c.context);
    // Everything create allocates: caches, split Q6_K copies, activation
    // buffers and logits, RoPE tables, workspaces and chained records.
    const uint64_t buffer_bytes =
        sizeof(float) * (T * (5ull * c.dim + 2ull * kv + 2ull * c.hidden + c.vocab) + 2ull * c.context * half +
                         T * (c.dim / 256)) +
        ws + m->attn_ws_bytes + qk_argmax_rows_workspace_bytes(c.vocab, max_tokens) + 2 * rec_bytes +
        T * (3 * sizeof(int32_t) + sizeof(qk_batch_token));
    if (int st0 = check_free_memory("qk_llama_batch_create",
                                    2 * cache * sizeof(float) + split_copy_bytes(*w, c, m->kv_dim) + buffer_bytes)) {
        delete m;
        return st0;
    }
    int st = QK_OK;
    if ((st = dev_alloc(m->mem.buffers, &m->x, T * c.dim, "residual")) || (st = dev_alloc(m->mem.buffers, &m->xn, T * c.dim, "normalized state")) ||
        (st = dev_alloc(m->mem.buffers, &m->q, T * c.dim, "query")) || (st = dev_alloc(m->mem.buffers, &m->k, T * kv, "key")) ||
        (st = dev_alloc(m->mem.buffers, &m->v, T * kv, "value")) || (st = dev_alloc(m->mem.buffers, &m->attn, T * c.dim, "attention")) ||
        (st = dev_alloc(m->mem.buffers, &m->tmp, T * c.dim, "residual update")) || (st = dev_alloc(m->mem.buffers, &m->gate, T * c.hidden, "gate")) ||
        (st = dev_alloc(m->mem.buffers, &m->up, T * c.hidden, "up projection")) ||
        (st = dev_alloc(m->mem.buffers, &m->logits, T * c.vocab, "logits")) ||
        (st = dev_alloc(m->mem.kv_cache, &m->key_cache, cache, "key cache")) ||
        (st = dev_alloc(m->mem.kv_cache, &m->value_cache, cache, "value cache")) ||
        (st = dev_alloc(m->mem.buffers, &m->cosine, static_cast<size_t>(c.context) * half, "RoPE cosine")) ||
        (st = dev_alloc(m->mem.buffers, &m->sine, static_cast<size_t>(c.context) * half, "RoPE sine")) ||
        (ws && (st = dev_alloc(m->mem.buffers, reinterpret_cast<uint8_t **>(&m->gemm_ws), ws, "matrix workspace"))) ||
        (m->attn_ws_bytes &&
         (st = dev_alloc(m->mem.buffers, reinterpret_cast<uint8_t **>(&m->attn_ws), m->attn_ws_bytes, "attention workspace"))) ||
        (st = dev_alloc(m->mem.buffers, reinterpret_cast<uint8_t **>(&m->argmax_ws), qk_argmax_rows_workspace_bytes(c.vocab, max_tokens),
                        "argmax workspace")) ||
        (st = dev_alloc(m->mem.buffers, &m->d_tokens, T, "input tokens")) || (st = dev_alloc(m->mem.buffers, &m->d_next, T, "next tokens")) ||
        (st = dev_alloc(m->mem.buffers, &m->d_rows, T, "logit rows")) || (st = dev_alloc(m->mem.buffers, &m->d_desc, T, "batch descriptor")) ||
        (rec_bytes && ((st = dev_alloc(m->mem.buffers, &m->rec_a, rec_bytes, "chained records")) ||
                       (st = dev_alloc(m->mem.buffers, &m->rec_b, rec_bytes, "chained records")) ||
                       (st = dev_alloc(m->mem.buffers, &m->ss, T * (c.dim / 256), "chained sums of squares"))))) {
        release_batch(m);
        return st;
    }
    if (hipHostMalloc(reinterpret_cast<void **>(&m->h_stage), stage_bytes(max_tokens), hipHostMallocDefault) !=
        hipSuccess) {
        release_batch(m);
        return qk::fail(QK_ERR_DEVICE, "qk_llama_batch_create: cannot allocate pinned staging");
    }
    std::vector<float> cosines(static_cast<size_t>(c.context) * half), sines(cosines.size()), freq(half);
    for (int i = 0; i < half; ++i) freq[i] = std::pow(c.rope_theta, -2.f * static_cast<float>(i) / head_dim);
    for (int pos = 0; pos < c.context; ++pos)
        for (int i = 0; i < half; ++i) {
            const float angle = static_cast<float>(pos) * freq[i];
            cosines[static_cast<size_t>(pos) * half + i] = std::cos(angle);
            sines[static_cast<size_t>(pos) * half + i] = std::sin(angle);
        }
    if (hipMemcpy(m->cosine, cosines.data(), cosines.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->sine, sines.data(), sines.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(m->key_cache, 0, cache * sizeof(float)) != hipSuccess ||
        hipMemset(m->value_cache, 0, cache * sizeof(float)) != hipSuccess) {
        release_batch(m);
        return qk::fail(QK_ERR_DEVICE, "qk_llama_batch_create: table upload failed");
    }
    if ((st = split_weights(m->owned, m->mem.weight_copies, m->w, m->layers, c, m->kv_dim, m->stream))) {
        release_batch(m);
        return st;
    }
    m->w.layers = m->layers.data();
    *out = m;
    return qk::ok();
}

int qk_llama_batch_destroy(qk_llama_batch *m) {
    if (!m) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_destroy: null handle");
    (void)hipStreamSynchronize(m->stream);
    release_batch(m);
    return qk::ok();
}

int qk_llama_batch_kv_cache(qk_llama_batch *m, float **key_cache, float **value_cache) {
    if (!m || !key_cache || !value_cache)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_kv_cache: null argument");
    *key_cache = m->key_cache;
    *value_cache = m->value_cache;
    return qk::ok();
}

int qk_llama_batch_memory_bytes(const qk_llama_batch *m, qk_llama_memory *out) {
    if (!m || !out) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_memory_bytes: null argument");
    *out = m->mem;
    return qk::ok();
}

int qk_llama_batch_logits(qk_llama_batch *m, const float **logits) {
    if (!m || !logits) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_logits: null argument");
    *logits = m->logits;
    return qk::ok();
}

int qk_llama_batch_set_trace(qk_llama_batch *m, float *residuals, int8_t *quantized) {
    if (!m) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_set_trace: null handle");
    if ((residuals && !qk::aligned(residuals, 4)))
        return qk::fail(QK_ERR_ALIGN, "qk_llama_batch_set_trace: residuals must be 4-byte aligned");
    m->trace_x = residuals;
    m->trace_q = quantized;
    return qk::ok();
}

int qk_llama_batch_matrix_calls(const qk_llama_batch *m, uint64_t *calls) {
    if (!m || !calls) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_matrix_calls: null argument");
    *calls = m->matrix_calls;
    return qk::ok();
}

int qk_llama_batch_residual(qk_llama_batch *m, const float **x) {
    if (!m || !x) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_residual: null argument");
    *x = m->x;
    return qk::ok();
}

int qk_llama_batch_forward_rows(qk_llama_batch *m, const int32_t *tokens, const qk_batch_token *desc, int n_tokens,
                                const int32_t *logit_rows, int n_rows, int32_t *next_tokens) {
    if (!m || !tokens || !desc || (n_rows > 0 && (!logit_rows || !next_tokens)))
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: null argument");
    const qk_llama_config &c = m->cfg;
    if (n_tokens < 1 || n_tokens > m->max_tokens)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: token count outside 1..max_tokens");
    if (n_rows < 0 || n_rows > n_tokens)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: logit row count outside 0..n_tokens");
    int max_pos = 0;
    int64_t rows = 0;
    for (int t = 0; t < n_tokens; ++t) {
        const qk_batch_token &d = desc[t];
        // kv_row + pos < cache_rows, written so a huge kv_row cannot overflow.
        if (tokens[t] < 0 || tokens[t] >= c.vocab || d.pos < 0 || d.pos >= c.context || d.kv_row < 0 ||
            d.kv_row > m->cache_rows - 1 - d.pos)
            return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: token " + std::to_string(t) +
                                                    " outside the vocabulary, the context or the cache");
        max_pos = std::max(max_pos, d.pos);
        rows += d.pos + 1;
    }
    bool identity = n_rows == n_tokens;   // logits of every token, in order
    for (int i = 0; i < n_rows; ++i) {
        if (logit_rows[i] < 0 || logit_rows[i] >= n_tokens)
            return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: logit row outside the batch");
        identity = identity && logit_rows[i] == i;
    }
    bool chained = false;
    int st;
    if ((st = check_kv_rows(desc, n_tokens, m->kv_writes, &chained))) return st;
    hipStream_t s = m->stream;
    const int T = n_tokens, dim = c.dim, kv = m->kv_dim, hd = m->head_dim;
    int32_t *h_tokens = reinterpret_cast<int32_t *>(m->h_stage);
    int32_t *h_next = h_tokens + m->max_tokens;
    int32_t *h_rows = h_next + m->max_tokens;
    qk_batch_token *h_desc = reinterpret_cast<qk_batch_token *>(h_rows + m->max_tokens);
    // The pinned staging is reused: the previous step's copies must be done.
    if (hipStreamSynchronize(s) != hipSuccess) return qk::fail(QK_ERR_DEVICE, "qk_llama_batch_forward: stream error");
    std::copy(tokens, tokens + T, h_tokens);
    std::copy(desc, desc + T, h_desc);
    if (n_rows) std::copy(logit_rows, logit_rows + n_rows, h_rows);
    if (hipMemcpyAsync(m->d_tokens, h_tokens, T * sizeof(int32_t), hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(m->d_desc, h_desc, T * sizeof(qk_batch_token), hipMemcpyHostToDevice, s) != hipSuccess ||
        (n_rows && !identity &&
         hipMemcpyAsync(m->d_rows, h_rows, n_rows * sizeof(int32_t), hipMemcpyHostToDevice, s) != hipSuccess))
        return qk::fail(QK_ERR_DEVICE, "qk_llama_batch_forward: batch upload failed");
    void *ws = m->gemm_ws;
    const size_t wsb = m->gemm_ws_bytes;
    // Seven products per layer and token, one LM-head product per logit row
    // (the reference's batched prefill counts 3, 1, 2 and 1 per token and
    // layer, inferencer.cu:1321, 1368, 1277).
    m->matrix_calls += 7ull * c.layers * T + n_rows;
    if ((st = qk_embedding(m->w.embd_type, m->w.token_embd, m->d_tokens, T, m->x, dim, c.vocab, s))) return st;
    // Per layer: fused QKV (RMSNorm staged), RoPE + KV write + attention,
    // o (+ residual), fused gate/up (RMSNorm staged), down (SiLU * up staged,
    // + residual).  When tokens of the step read rows that other tokens of
    // it write (a prefill chunk), RoPE and the KV write run as a launch of
    // their own before the attention, as rope_cache_batch_cuda precedes
    // attention_batch_cuda (inferencer.cu:953-1041): every token then sees
    // the rows of the tokens before it and none after (causal).
    qk::GemvFusion attn_in, ffn_in, residual, down_in;
    attn_in.norm_eps = ffn_in.norm_eps = c.eps;
    residual.accumulate = down_in.accumulate = 1;
    down_in.up = m->up;
    qk::SplitAttention attn{};
    attn.q = m->q;
    attn.k = chained ? nullptr : m->k;
    attn.v = chained ? nullptr : m->v;
    attn.cosine = m->cosine;
    attn.sine = m->sine;
    attn.key_cache = m->key_cache;
    attn.head_major = 1;
    attn.value_cache = m->value_cache;
    attn.out = m->attn;
    attn.desc = m->d_desc;
    attn.cache_rows = m->cache_rows;
    attn.rows_hint = rows;
    attn.max_pos = max_pos;
    attn.n_tokens = T;
    attn.heads = c.heads;
    attn.kv_heads = c.kv_heads;
    attn.head_dim = hd;
    // From 8 tokens on (matrix cores) the projections chain: attention packs
    // its outputs as o's records, o's reduction adds the residual and packs
    // x * ffn_norm for gate/up (sums of squares for the deferred RMSNorm),
    // gate/up's packs SiLU(gate) * up for down, down's adds the residual and
    // packs x * the next attn_norm for the next QKV -- nine launches per
    // layer (one more with split attention) instead of thirteen.
    const bool chain = qk::batched_chain_supported(T) && m->rec_a;
    const bool attn_records = chain && qk::attention_gemm_records(attn);
    bool head_normed = false;
    if (m->int8 && (st = batch_layers_int8(m, T, chained, attn, s, n_rows && identity ? m->w.output_norm : nullptr,
                                           &head_normed)))
        return st;
    for (int l = 0; l < c.layers && !m->int8; ++l) {
        const qk_llama_layer &L = m->layers[l];
        attn_in.norm_w = L.attn_norm;
        ffn_in.norm_w = L.ffn_norm;
        const qk_matrix qkv[3] = {{L.q_type, dim, L.q, m->q}, {L.k_type, kv, L.k, m->k}, {L.v_type, kv, L.v, m->v}};
        qk::GemvFusion qkv_in = attn_in;
        if (chain && l > 0) {
            qkv_in = qk::GemvFusion{};
            qkv_in.in_records = m->rec_a;
            qkv_in.in_ss = m->ss;
            qkv_in.norm_eps = c.eps;
        }
        if ((st = qk::launch_batched_fused(qkv, 3, m->x, dim, dim, T, qkv_in, ws, wsb, s))) return st;
        if (chained &&
            (st = qk::launch_rope_kv_batched(m->q, m->k, m->v, m->cosine, m->sine, m->key_cache, m->value_cache, l,
                                             m->cache_rows, m->d_desc, T, c.context, c.heads, c.kv_heads, hd, 1, s)))
            return st;
        attn.layer = l;
        // In the chain, attention packs the o projection's records itself
        // (rec_b is free: down read it in the previous layer).
        attn.gemm_rec = chain && attn_records ? m->rec_b : nullptr;
        if ((st = qk::launch_split_attention(attn, 0, m->attn_ws, m->attn_ws_bytes, s))) return st;
        const qk_matrix o{L.o_type, dim, L.o, m->x};
        const qk_matrix gu[2] = {{L.gate_type, c.hidden, L.gate, m->gate}, {L.up_type, c.hidden, L.up, m->up}};
        const qk_matrix down{L.down_type, dim, L.down, m->x};
        if (!chain) {
            if ((st = qk::launch_batched_fused(&o, 1, m->attn, dim, dim, T, residual, ws, wsb, s)) ||
                (st = qk::launch_batched_fused(gu, 2, m->x, dim, dim, T, ffn_in, ws, wsb, s)) ||
                (st = qk::launch_batched_fused(&down, 1, m->gate, c.hidden, c.hidden, T, down_in, ws, wsb, s)) ||
                (st = batch_trace_x(m, l, T, s)))
                return st;
            continue;
        }
        qk::GemvFusion o_f = residual, gu_f, down_f;
        if (attn_records) o_f.in_records = m->rec_b;
        o_f.out_records = m->rec_a;
        o_f.out_gain = L.ffn_norm;
        o_f.out_ss = m->ss;
        gu_f.in_records = m->rec_a;
        gu_f.in_ss = m->ss;
        gu_f.norm_eps = c.eps;
        gu_f.pair = 1;
        gu_f.out_records = m->rec_b;
        down_f.in_records = m->rec_b;
        down_f.accumulate = 1;
        if (l + 1 < c.layers) {
            down_f.out_records = m->rec_a;
            down_f.out_gain = m->layers[l + 1].attn_norm;
            down_f.out_ss = m->ss;
        }
        if ((st = qk::launch_batched_fused(&o, 1, m->attn, dim, dim, T, o_f, ws, wsb, s)) ||
            (st = qk::launch_batched_fused(gu, 2, m->x, dim, dim, T, gu_f, ws, wsb, s)) ||
            (st = qk::launch_batched_fused(&down, 1, m->gate, c.hidden, c.hidden, T, down_f, ws, wsb, s)) ||
            (st = batch_trace_x(m, l, T, s)))
            return st;
    }
    if (!n_rows) return qk::ok();
    // The LM head over the selected tokens only (the reference's prefill
    // computes the chunk's last token, inferencer.cu:1410-1414): their rows
    // of x are gathered first unless the selection is every token in order.
    const float *head_x = m->x;
    if (!identity) {
        if ((st = qk::launch_gather_rows(m->x, dim, m->d_rows, n_rows, dim, m->tmp, s))) return st;
        head_x = m->tmp;
    }
    qk::GemvFusion out_in;
    out_in.norm_w = m->w.output_norm;
    out_in.norm_eps = c.eps;
    const void *out_w = m->w.output ? m->w.output : m->w.token_embd;
    const int out_type = m->w.output ? m->w.output_type : m->w.embd_type;
    const qk_matrix head{out_type, c.vocab, out_w, m->logits};
    if (m->int8) {
        // rmsnorm_cuda, then gpu.matvec's quantization and INT8 product
        // (inferencer.cu:1408-1414) for the selected rows.
        // Over the GGUF-block copy of a Q6_K head (head_q6k).
        const qk_matrix head_i8 = m->head_q6k ? qk_matrix{QK_TYPE_Q6_K, c.vocab, m->head_q6k, m->logits} : head;
        if ((!head_normed && (st = qk_rmsnorm_quantize_x32(head_x, dim, m->w.output_norm, nullptr, 0, m->xq, dim, m->xs,
                                                           dim / 32, dim, n_rows, c.eps, s))) ||
            (st = batch_gemm_i8(m, &head_i8, 1, m->xq, m->xs, dim, n_rows, false, s)))
            return st;
    } else if ((st = qk::launch_batched_fused(&head, 1, head_x, dim, dim, n_rows, out_in, ws, wsb, s))) {
        return st;
    }
    if ((st = qk_argmax_rows_f32(m->logits, c.vocab, c.vocab, n_rows, m->d_next, m->argmax_ws, s))) return st;
    if (hipMemcpyAsync(h_next, m->d_next, n_rows * sizeof(int32_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return qk::fail(QK_ERR_DEVICE, "qk_llama_batch_forward: next token download failed");
    std::copy(h_next, h_next + n_rows, next_tokens);
    return qk::ok();
}

int qk_llama_batch_forward(qk_llama_batch *m, const int32_t *tokens, const qk_batch_token *desc, int n_tokens,
                           int need_logits, int32_t *next_tokens) {
    if (!m) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: null handle");
    if (need_logits && !next_tokens) return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: null argument");
    if (!need_logits) return qk_llama_batch_forward_rows(m, tokens, desc, n_tokens, nullptr, 0, nullptr);
    if (n_tokens < 1 || n_tokens > m->max_tokens)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_llama_batch_forward: token count outside 1..max_tokens");
    std::vector<int32_t> all(n_tokens);
    for (int t = 0; t < n_tokens; ++t) all[t] = t;
    return qk_llama_batch_forward_rows(m, tokens, desc, n_tokens, all.data(), n_tokens, next_tokens);
}

}  // extern "C"
