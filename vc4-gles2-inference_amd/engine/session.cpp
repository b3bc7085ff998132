// The decode engine: weights from an MMCF container uploaded through libvgx,
// the reference's fused GPU layer loop (Session::forward_gpu_hidden,
// engine/src/session.cpp:1459-1584) issued as libvgx launches on one stream,
// and greedy generation with the token kept on the device.
#include <hip/hip_runtime.h>
#include <sys/stat.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <string>
#include <vector>

#include "engine_err.h"
#include "mmcf_reader.h"
#include "vgx.h"
#include "vgx_engine.h"

namespace {

thread_local std::string g_err;

int fail(int st, const std::string& msg) {
    g_err = msg;
    return st;
}

}  // namespace

int engine_fail(int status, const std::string& msg) { return fail(status, msg); }
void engine_clear_error() { g_err.clear(); }
const std::string& engine_error() { return g_err; }

struct vgx_engine {
    vgxe::Container c;
    vgxe::ModelMeta m;
    vgx_ctx* ctx = nullptr;
    vgx_attn* attn = nullptr;
    vgx_conv* conv = nullptr;  // LFM2 conv-layer state (hybrid models only)
    struct Layer {
        vgx_mat *qkv = nullptr, *wo = nullptr, *w1 = nullptr, *w3 = nullptr, *w2 = nullptr;
        vgx_mat *conv_in = nullptr, *conv_out = nullptr;  // conv layers instead of qkv / wo
        int16_t *rms_att = nullptr, *rms_ffn = nullptr;
        int hs = 0;
    };
    std::vector<Layer> L;
    std::vector<vgx_mat*> head_tiles;
    vgx_group* head = nullptr;
    vgx_attn_desc attn_desc{};  // with the host tables it points into
    std::vector<float> rope_c, rope_s;
    std::vector<uint8_t> attn_flag;
    int8_t* emb = nullptr;
    float* emb_scale = nullptr;
    int16_t *h = nullptr, *x1 = nullptr, *qkv = nullptr, *att = nullptr, *hbuf = nullptr;
    int16_t *logits = nullptr, *rms_final = nullptr;
    int* toks = nullptr;  // device token slots: [0, seq) prompt/decode history, [seq] the host step's
    int seq = 0, kv_bits = 16, ffn_chunk = 0;
    // batched prefill: row buffers for up to pcap positions; prompts run in
    // batches of pbatch (serial steps when pbatch < 2)
    int pcap = 0, pbatch = 0;
    int16_t *bh = nullptr, *bx1 = nullptr, *bxn = nullptr, *bqkv = nullptr, *batt = nullptr, *bhid = nullptr;
    // batched decode of nseq sequences in lockstep: their KV caches, the LM
    // head as one matrix, nseq rows of logits, the token history
    vgx_attn* attn_b = nullptr;
    int nseq_b = 0;
    vgx_mat* head_cat = nullptr;
    int16_t* blog = nullptr;
    int* btok = nullptr;
    size_t btok_cap = 0;
    std::vector<void*> allocs;
    // the container's identity, as the prefix cache header records it
    uint64_t src_size = 0, src_mtime = 0;
    // the greedy decode step as one HIP graph, replayed per token: the token
    // and the position live in device memory (tok_cur, pos_dev) and the step
    // ends by appending the token to the history and advancing the position
    bool use_graph = true;
    hipGraph_t step_graph = nullptr;
    hipGraphExec_t step_exec = nullptr;
    // the same step captured kMultiSteps times in one graph (multi_exec), for
    // runs of that many tokens, where a step has at most kMultiMaxNodes
    // launches: each replayed graph costs a few microseconds of its own at its
    // boundary (MiniMind3 q8, 42 launches a step: 5950 -> 6109 tokens/s with 4
    // steps a graph, 6064 with 2, 6106 with 8; the LFM2.5-shaped hybrid, 82: 3160
    // -> 3221), but the 0.5B t3 step (122 launches) ran 0.3-0.6% slower in
    // graphs of 2, 4 or 8 steps
    static constexpr int kMultiSteps = 4;
    static constexpr size_t kMultiMaxNodes = 100;
    hipGraph_t multi_graph = nullptr;
    hipGraphExec_t multi_exec = nullptr;
    int *pos_dev = nullptr, *tok_cur = nullptr;
    int pos_host = 0;
    // the candidate pass: its per-chunk records (device and host); valid when
    // every LM-head tile but the last has a multiple of 16 rows, so the
    // reference's per-tile chunks are 16-chunks of the concatenated logits
    bool cand_tiles_ok = true;
    int* chunk_dev = nullptr;
    std::vector<int> chunk_host;
    std::vector<int16_t> logits_tmp;

    ~vgx_engine() {
        if (step_exec) (void)hipGraphExecDestroy(step_exec);
        if (step_graph) (void)hipGraphDestroy(step_graph);
        if (multi_exec) (void)hipGraphExecDestroy(multi_exec);
        if (multi_graph) (void)hipGraphDestroy(multi_graph);
        for (auto& l : L) {
            vgx_mat_free(l.qkv); vgx_mat_free(l.wo); vgx_mat_free(l.w1); vgx_mat_free(l.w3); vgx_mat_free(l.w2);
            vgx_mat_free(l.conv_in); vgx_mat_free(l.conv_out);
        }
        vgx_group_free(head);
        for (vgx_mat* t : head_tiles) vgx_mat_free(t);
        vgx_mat_free(head_cat);
        vgx_attn_free(attn_b);
        vgx_attn_free(attn);
        vgx_conv_free(conv);
        for (void* p : allocs) (void)hipFree(p);
        vgx_ctx_destroy(ctx);
    }

    template <typename T>
    int dalloc(T** p, size_t n) {
        void* q = nullptr;
        hipError_t e = hipMalloc(&q, n * sizeof(T) + 16);
        if (e != hipSuccess) return fail(VGX_ENOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
        allocs.push_back(q);
        *p = static_cast<T*>(q);
        return VGX_OK;
    }

    template <typename T>
    int upload(T** p, const T* src, size_t n) {
        int st = dalloc(p, n);
        if (st) return st;
        hipError_t e = hipMemcpy(*p, src, n * sizeof(T), hipMemcpyHostToDevice);
        return e == hipSuccess ? VGX_OK : fail(VGX_EHIP, hipGetErrorString(e));
    }

    // One weight matrix (rows r0..r1 of the record) through vgx_mat_upload:
    // GPU::upload's job (engine/src/gpu_upload.cpp:20-192), the bytes as the
    // container holds them.
    int upload_mat(int kind, int layer, int r0, int r1, float scale_mul, vgx_mat** out) {
        const vgxe::Record* r = c.find(kind, layer, 0);
        if (!r) return fail(VGX_EINVAL, "missing tensor kind 0x" + std::to_string(kind) + " layer " + std::to_string(layer));
        if (r1 < 0) r1 = (int)r->rows;
        const vgxe::Record* plane = c.find(kind, layer, 3);
        vgx_weight_desc d{};
        d.rows = r1 - r0;
        d.cols = (int)r->cols;
        d.scale = r->scale;
        d.scale_mul = scale_mul;
        if (plane && (plane->rows != r->rows || plane->bytes != (uint64_t)r->rows * 4))
            return fail(VGX_EINVAL, "row plane does not match its matrix");
        d.row_plane = plane ? reinterpret_cast<const float*>(plane->body) + r0 : nullptr;
        switch (r->dtype) {
            case vgxe::DT_Q8U8:
            case vgxe::DT_Q8I8:
                d.kind = VGX_Q8;
                d.prebiased = r->dtype == vgxe::DT_Q8U8;
                d.body = r->body + (size_t)r0 * r->cols;
                d.body_bytes = (size_t)d.rows * r->cols;
                break;
            case vgxe::DT_Q4: {
                const vgxe::Record* s = c.find(kind, layer, 1);
                const vgxe::Record* mn = c.find(kind, layer, 2);
                if (!s || !mn) return fail(VGX_EINVAL, "q4 matrix without its scale/min planes");
                const size_t g = r->cols / 32;
                d.kind = VGX_Q4;
                d.body = r->body + (size_t)r0 * (r->cols / 2);
                d.body_bytes = (size_t)d.rows * (r->cols / 2);
                d.q4_scale = reinterpret_cast<const int16_t*>(s->body) + (size_t)r0 * g;
                d.q4_min = reinterpret_cast<const int16_t*>(mn->body) + (size_t)r0 * g;
                break;
            }
            case vgxe::DT_T3: {
                if (r0 % 2) return fail(VGX_EINVAL, "t3 row slice off a row pair");
                const size_t stride = (size_t)((r->cols + 7) / 8) * 4;
                d.kind = VGX_T3;
                d.body = r->body + (size_t)(r0 / 2) * stride;
                d.body_bytes = (size_t)((d.rows + 1) / 2) * stride;
                break;
            }
            default:
                return fail(VGX_EINVAL, "tensor dtype " + std::to_string(r->dtype) + " is not a kernel matrix");
        }
        return vgx_mat_upload(ctx, &d, out);
    }

    bool is_conv(int l) const { return !m.layer_conv.empty() && m.layer_conv[l]; }

    int init(int device, int seq_req, int kv_req) {
        m = c.meta();
        if (!m.layer_conv.empty() && (int)m.layer_conv.size() != m.layers)
            return fail(VGX_EINVAL, "layer types (key 14) do not match the layer count");
        seq = seq_req > 0 ? seq_req : m.seq;
        kv_bits = kv_req;
        if (kv_bits != 16 && kv_bits != 8) return fail(VGX_EINVAL, "kv_bits must be 16 or 8");
        int st = vgx_ctx_create(device, &ctx);
        if (st) return fail(st, vgx_last_error());
        // split_ffn (engine/src/model.cpp:246-266): two chunks over 2048
        ffn_chunk = m.hidden > 2048 ? (m.hidden + 1) / 2 : 0;
        const int D = m.dim, hd = m.head_dim();
        L.resize(m.layers);
        std::vector<int16_t> q16(D);
        const vgxe::Record* ra = c.find(vgxe::T_RMS_ATT);
        const vgxe::Record* rf = c.find(vgxe::T_RMS_FFN);
        const vgxe::Record* rfin = c.find(vgxe::T_RMS_FINAL);
        if (ra->bytes != (uint64_t)m.layers * D * 4 || rf->bytes != ra->bytes || rfin->bytes != (uint64_t)D * 4)
            return fail(VGX_EINVAL, "rms weight shapes");
        // LFM2 conv layers (key 14): in_proj 3*dim x dim, the f32 depthwise
        // kernel dim x 3, out_proj dim x dim (engine/src/model.cpp:1142-1160,
        // 1480-1500)
        std::vector<float> conv_w;
        std::vector<uint8_t> conv_flag((size_t)m.layers, 0);
        bool hybrid = false;
        for (int l = 0; l < m.layers; ++l) {
            Layer& ly = L[l];
            ly.hs = m.hid_scale.empty() ? 0 : m.hid_scale[l];
            if (is_conv(l)) {
                const vgxe::Record* kw = c.find(vgxe::T_CONV_W, l);
                if (!kw || kw->dtype != vgxe::DT_F32 || kw->rows != (uint32_t)D || kw->cols != 3)
                    return fail(VGX_EINVAL, "layer " + std::to_string(l) + ": the conv kernel must be f32 dim x 3");
                if ((st = upload_mat(vgxe::T_CONV_IN, l, 0, -1, 0.0f, &ly.conv_in))) return st;
                if ((st = upload_mat(vgxe::T_CONV_OUT, l, 0, -1, 0.0f, &ly.conv_out))) return st;
                int kind, rows, cols;
                vgx_mat_shape(ly.conv_in, &kind, &rows, &cols);
                if (rows != 3 * D || cols != D) return fail(VGX_EINVAL, "conv in_proj must be 3*dim x dim");
                vgx_mat_shape(ly.conv_out, &kind, &rows, &cols);
                if (rows != D || cols != D) return fail(VGX_EINVAL, "conv out_proj must be dim x dim");
                conv_w.resize((size_t)m.layers * D * 3, 0.0f);
                std::memcpy(conv_w.data() + (size_t)l * D * 3, kw->body, (size_t)D * 3 * 4);
                conv_flag[l] = 1;
                hybrid = true;
            } else {
                if ((st = upload_mat(vgxe::T_QKV, l, 0, -1, 0.0f, &ly.qkv))) return st;
                if ((st = upload_mat(vgxe::T_WO, l, 0, -1, 0.0f, &ly.wo))) return st;
            }
            if (c.find(vgxe::T_W13, l)) {
                if ((st = upload_mat(vgxe::T_W13, l, 0, m.hidden, 0.0f, &ly.w1))) return st;
                if ((st = upload_mat(vgxe::T_W13, l, m.hidden, 2 * m.hidden, 0.0f, &ly.w3))) return st;
            } else {
                if ((st = upload_mat(vgxe::T_W1, l, 0, -1, 0.0f, &ly.w1))) return st;
                if ((st = upload_mat(vgxe::T_W3, l, 0, -1, 0.0f, &ly.w3))) return st;
            }
            // Model::apply_hidden_scale (engine/src/model.cpp:407-429)
            if ((st = upload_mat(vgxe::T_W2, l, 0, -1, ly.hs ? (float)(1u << ly.hs) : 0.0f, &ly.w2))) return st;
            // the norm vectors on the q16 grid (make_q16_pair_texture = x_pack)
            vgx_quantize_act(reinterpret_cast<const float*>(ra->body) + (size_t)l * D, D, q16.data());
            if ((st = upload(&ly.rms_att, q16.data(), D))) return st;
            vgx_quantize_act(reinterpret_cast<const float*>(rf->body) + (size_t)l * D, D, q16.data());
            if ((st = upload(&ly.rms_ffn, q16.data(), D))) return st;
        }
        vgx_quantize_act(reinterpret_cast<const float*>(rfin->body), D, q16.data());
        if ((st = upload(&rms_final, q16.data(), D))) return st;
        if (hybrid) {
            conv_w.resize((size_t)m.layers * D * 3, 0.0f);
            if ((st = vgx_conv_create(ctx, D, m.layers, 3, conv_w.data(), conv_flag.data(), &conv))) return st;
        }
        // embedding (signed q8 rows + f32 row scales)
        const vgxe::Record* e = c.find(vgxe::T_EMB);
        const vgxe::Record* es = c.find(vgxe::T_EMB_SCALE);
        if (e->dtype != vgxe::DT_Q8I8 || e->rows != (uint32_t)m.vocab || e->cols != (uint32_t)D ||
            es->bytes != (uint64_t)m.vocab * 4)
            return fail(VGX_EINVAL, "this engine reads q8 embedding rows");
        if ((st = upload(&emb, reinterpret_cast<const int8_t*>(e->body), (size_t)m.vocab * D))) return st;
        if ((st = upload(&emb_scale, reinterpret_cast<const float*>(es->body), (size_t)m.vocab))) return st;
        // LM head: the logits tiles, or the embedding rows for a dedup head
        // (engine/src/model.cpp:1566-1586)
        for (int i = 0; c.find(vgxe::T_LOGITS, i); ++i) {
            vgx_mat* t = nullptr;
            if ((st = upload_mat(vgxe::T_LOGITS, i, 0, -1, 0.0f, &t))) return st;
            if (c.find(vgxe::T_LOGITS, i + 1) && c.find(vgxe::T_LOGITS, i)->rows % 16 != 0) cand_tiles_ok = false;
            head_tiles.push_back(t);
        }
        if (head_tiles.empty()) {
            const float* s = reinterpret_cast<const float*>(es->body);
            float unit = 0.0f;
            for (int v = 0; v < m.vocab; ++v) unit = s[v] > unit ? s[v] : unit;
            if (unit <= 0.0f) return fail(VGX_EINVAL, "a dedup head needs embedding scales");
            for (int st0 = 0; st0 < m.vocab; st0 += 1536) {
                const int rows = m.vocab - st0 < 1536 ? m.vocab - st0 : 1536;
                std::vector<float> plane(rows);
                for (int k = 0; k < rows; ++k) plane[k] = s[st0 + k] / unit;
                vgx_weight_desc d{};
                d.kind = VGX_Q8; d.rows = rows; d.cols = D; d.prebiased = 0; d.scale = unit;
                d.body = e->body + (size_t)st0 * D; d.body_bytes = (size_t)rows * D; d.row_plane = plane.data();
                vgx_mat* t = nullptr;
                if ((st = vgx_mat_upload(ctx, &d, &t))) return st;
                head_tiles.push_back(t);
            }
        }
        if ((st = vgx_group_create(ctx, (int)head_tiles.size(), head_tiles.data(), &head))) return st;
        // the logits buffers hold vocab rows and a token id indexes the
        // concatenated tiles, so the tiles must cover exactly the vocabulary
        if (vgx_group_rows(head) != m.vocab)
            return fail(VGX_EINVAL, "the logits tiles hold " + std::to_string(vgx_group_rows(head)) +
                                        " rows for a vocabulary of " + std::to_string(m.vocab));
        // attention state: Session's rope tables (engine/src/session.cpp:188-202)
        const int half = hd / 2;
        std::vector<float>& rc = rope_c;
        std::vector<float>& rs = rope_s;
        rc.assign((size_t)seq * half, 0.0f);
        rs.assign((size_t)seq * half, 0.0f);
        for (int p = 0; p < seq; ++p)
            for (int i = 0; i < half; ++i) {
                float freq = 1.0f / powf(m.theta, (2.0f * i) / hd);
                float a = p * freq;
                rc[(size_t)p * half + i] = cosf(a);
                rs[(size_t)p * half + i] = sinf(a);
            }
        vgx_attn_desc& ad = attn_desc;
        ad = vgx_attn_desc{};
        ad.dim = D; ad.heads = m.heads; ad.kv_heads = m.kv_heads; ad.head_dim = hd; ad.seq = seq;
        ad.layers = m.layers; ad.kv_bits = kv_bits; ad.rope_half = m.rope_half; ad.qk_norm = m.qk_norm;
        ad.rope_cos = rc.data(); ad.rope_sin = rs.data();
        if (m.qk_norm) {
            const vgxe::Record* qn = c.find(vgxe::T_Q_NORM);
            const vgxe::Record* kn = c.find(vgxe::T_K_NORM);
            if (!qn || !kn || qn->bytes != (uint64_t)m.layers * hd * 4 || kn->bytes != qn->bytes)
                return fail(VGX_EINVAL, "q/k norm weights missing or misshapen");
            ad.q_norm = reinterpret_cast<const float*>(qn->body);
            ad.k_norm = reinterpret_cast<const float*>(kn->body);
        }
        attn_flag.assign((size_t)m.layers, 0);
        for (int l = 0; l < m.layers; ++l) attn_flag[l] = is_conv(l) ? 0 : 1;
        ad.layer_is_attn = attn_flag.data();
        if ((st = vgx_attn_create(ctx, &ad, &attn))) return st;
        // the qkv rows, or a conv layer's in_proj rows (B, C, x)
        const int qkv_rows = D + 2 * m.kv_dim() > (hybrid ? 3 * D : 0) ? D + 2 * m.kv_dim() : 3 * D;
        if ((st = dalloc(&h, D)) || (st = dalloc(&x1, D)) || (st = dalloc(&att, D)) ||
            (st = dalloc(&qkv, qkv_rows)) || (st = dalloc(&hbuf, m.hidden)) ||
            (st = dalloc(&logits, (size_t)m.vocab)) || (st = dalloc(&toks, (size_t)seq + 1)))
            return st;
        pcap = seq < 512 ? seq : 512;
        pbatch = pcap;
        const size_t P = (size_t)pcap;
        if ((st = dalloc(&bh, P * D)) || (st = dalloc(&bx1, P * D)) || (st = dalloc(&bxn, P * D)) ||
            (st = dalloc(&batt, P * D)) || (st = dalloc(&bqkv, P * qkv_rows)) || (st = dalloc(&bhid, P * m.hidden)))
            return st;
        hipError_t he = hipDeviceSynchronize();
        return he == hipSuccess ? VGX_OK : fail(VGX_EHIP, hipGetErrorString(he));
    }

    // Session::forward_gpu_hidden for one position; the token is read from
    // device memory.  With want_logits the final RMSNorm, the LM head and the
    // argmax (into *next_dev) follow.  Each RMSNorm runs inside the GEMV that
    // consumes it (the attention norm in the qkv draw, the FFN norm in the
    // gate, the final norm in the LM head with its argmax): five launches a
    // layer.
    // pos_dev: the position is read from device memory instead (the step a
    // graph replays; never position 0).
    // step_tail (the replayed step): h already holds the token's embedding,
    // and the argmax launch also advances *pos_dev, appends the token to the
    // history and embeds it into h for the next replay.
    int forward(const int* token_dev, int pos, bool want_logits, int* next_dev, vgx_attn* A,
                int* pos_dev = nullptr, bool step_tail = false) {
        int st;
        const int D = m.dim;
        const float eps = m.rms_eps;
        if (!pos_dev && pos == 0 && conv && (st = vgx_conv_reset(conv))) return st;  // a new sequence
        if (!step_tail && (st = vgx_embed_q8(ctx, emb, emb_scale, m.vocab, D, token_dev, h))) return st;
        for (int l = 0; l < m.layers; ++l) {
            Layer& ly = L[l];
            if (is_conv(l)) {
                // GPU::conv_block (engine/src/gpu_conv.cpp:165-225): in_proj,
                // the gated short conv, out_proj + residual
                if ((st = vgx_gemv_rms(ctx, ly.conv_in, h, ly.rms_att, eps, nullptr, qkv))) return st;
                if ((st = vgx_conv_step(conv, l, 1, qkv, att))) return st;
                if ((st = vgx_gemv(ctx, ly.conv_out, att, h, x1))) return st;
            } else {
                if ((st = vgx_gemv_rms(ctx, ly.qkv, h, ly.rms_att, eps, nullptr, qkv))) return st;
                st = pos_dev ? vgx_attn_block_at(A, l, pos_dev, qkv, att) : vgx_attn_block(A, l, pos, qkv, att);
                if (st) return st;
                if ((st = vgx_gemv(ctx, ly.wo, att, h, x1))) return st;
            }
            if ((st = vgx_ffn_gate_rms(ctx, ly.w1, ly.w3, x1, ly.rms_ffn, eps, ly.hs, hbuf))) return st;
            if (ffn_chunk) st = vgx_gemv_add_split(ctx, ly.w2, ffn_chunk, hbuf, x1, h);
            else st = vgx_gemv(ctx, ly.w2, hbuf, x1, h);
            if (st) return st;
        }
        if (!want_logits) return VGX_OK;
        if (step_tail)
            return vgx_logits_argmax_step(ctx, head, h, rms_final, eps, logits, next_dev, pos_dev, toks, seq, emb,
                                          emb_scale, m.vocab, D, h);
        return vgx_logits_argmax_rms(ctx, head, h, rms_final, eps, logits, next_dev);
    }

    // Batched prefill of positions pos0 .. pos0+n-1 (Session::step_group,
    // engine/src/session.cpp:1741-1795): the same layer sequence as forward()
    // over n rows at once -- GEMMs on the int8 matrix cores, the KV rows of all
    // n positions appended before any of them attends.  Every row is the exact
    // result of forward() on that position, so the logits of the last one are
    // identical to the serial loop's.
    int prefill(const int* toks_dev, int pos0, int n, bool want_logits, int* next_dev, vgx_attn* A) {
        int st;
        const int D = m.dim;
        const float eps = m.rms_eps;
        if (n <= 0 || n > pcap) return fail(VGX_EINVAL, "prefill: batch outside 1.." + std::to_string(pcap));
        if (pos0 == 0 && conv && (st = vgx_conv_reset(conv))) return st;  // a new sequence
        // RMSNorm in the consuming GEMM up to 32 positions (one token tile:
        // the normalisation runs once per row tile); above, on its own (the
        // first layer's in the embedding launch)
        const bool fuse = n <= 32;
        st = fuse ? vgx_embed_q8_batch(ctx, emb, emb_scale, m.vocab, D, n, toks_dev, bh)
                  : vgx_embed_q8_rms_batch(ctx, emb, emb_scale, m.vocab, D, n, toks_dev, bh, L[0].rms_att, eps, bxn);
        if (st) return st;
        for (int l = 0; l < m.layers; ++l) {
            Layer& ly = L[l];
            if (!fuse && l > 0 && (st = vgx_rmsnorm_batch(ctx, n, D, bh, ly.rms_att, eps, bxn))) return st;
            const vgx_mat* in_mat = is_conv(l) ? ly.conv_in : ly.qkv;
            st = fuse ? vgx_gemm_rms(ctx, in_mat, n, bh, ly.rms_att, eps, nullptr, bqkv)
                      : vgx_gemm(ctx, in_mat, n, bxn, nullptr, bqkv);
            if (st) return st;
            if (is_conv(l)) {
                // the conv over the batch walks its positions in order
                if ((st = vgx_conv_step(conv, l, n, bqkv, batt))) return st;
                if ((st = vgx_gemm(ctx, ly.conv_out, n, batt, bh, bx1))) return st;
            } else {
                if ((st = vgx_kv_append_batch(A, l, pos0, n, bqkv))) return st;
                if ((st = vgx_attn_decode_batch(A, l, pos0, n, bqkv, batt))) return st;
                if ((st = vgx_gemm(ctx, ly.wo, n, batt, bh, bx1))) return st;
            }
            if (fuse) {
                if ((st = vgx_ffn_gate_batch_rms(ctx, ly.w1, ly.w3, n, bx1, ly.rms_ffn, eps, ly.hs, bhid))) return st;
            } else {
                if ((st = vgx_rmsnorm_batch(ctx, n, D, bx1, ly.rms_ffn, eps, bxn))) return st;
                if ((st = vgx_ffn_gate_batch(ctx, ly.w1, ly.w3, n, bxn, ly.hs, bhid))) return st;
            }
            if (ffn_chunk) st = vgx_gemm_add_split(ctx, ly.w2, ffn_chunk, n, bhid, bx1, bh);
            else st = vgx_gemm(ctx, ly.w2, n, bhid, bx1, bh);
            if (st) return st;
        }
        if (!want_logits) return VGX_OK;
        return vgx_logits_argmax_rms(ctx, head, bh + (size_t)(n - 1) * D, rms_final, eps, logits, next_dev);
    }

    // The prompt tokens at toks_dev[0..n) for positions pos0.., in batches of
    // up to pbatch (one position at a time when pbatch < 2), on the KV cache A.
    int run_prompt(const int* toks_dev, int pos0, int n, int* next_dev, vgx_attn* A) {
        int st;
        if (pbatch < 2) {
            for (int p = 0; p < n; ++p)
                if ((st = forward(toks_dev + p, pos0 + p, p == n - 1, next_dev, A))) return st;
            return VGX_OK;
        }
        for (int p = 0; p < n; p += pbatch) {
            const int b = n - p < pbatch ? n - p : pbatch;
            if ((st = prefill(toks_dev + p, pos0 + p, b, p + b == n, next_dev, A))) return st;
        }
        return VGX_OK;
    }

    // The decode step captured once: forward() on the token at tok_cur (its
    // embedding already in h) and the position at pos_dev, its argmax back into
    // tok_cur, toks[pos + 1] = tok_cur, ++pos and the new token's embedding
    // into h, the last three in the argmax reduction's launch.  Every argument
    // is fixed, so one instantiation serves every token of every later
    // generation; the first replay needs h filled by the caller.
    int ensure_step_graph() {
        if (step_exec) return VGX_OK;
        int st;
        if (!pos_dev && ((st = dalloc(&pos_dev, 1)) || (st = dalloc(&tok_cur, 1)))) return st;
        if ((st = capture_steps(1, &step_graph, &step_exec))) return st;
        size_t nodes = 0;
        if (hipGraphGetNodes(step_graph, nullptr, &nodes) != hipSuccess) return fail(VGX_EHIP, "decode graph: nodes");
        if (nodes <= kMultiMaxNodes && (st = capture_steps(kMultiSteps, &multi_graph, &multi_exec))) return st;
        return VGX_OK;
    }

    // n consecutive decode steps captured into one graph and instantiated.
    int capture_steps(int n, hipGraph_t* graph, hipGraphExec_t* exec) {
        hipStream_t s = static_cast<hipStream_t>(vgx_ctx_stream(ctx));
        if (hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed) != hipSuccess)
            return fail(VGX_EHIP, "decode graph: begin capture");
        int st = VGX_OK;
        for (int k = 0; k < n && !st; ++k) st = forward(tok_cur, 0, true, tok_cur, attn, pos_dev, true);
        hipGraph_t g = nullptr;
        const hipError_t ec = hipStreamEndCapture(s, &g);
        if (st || ec != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return st ? st : fail(VGX_EHIP, std::string("decode graph: capture: ") + hipGetErrorString(ec));
        }
        hipGraphExec_t x = nullptr;
        const hipError_t ei = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
        if (ei != hipSuccess) {
            (void)hipGraphDestroy(g);
            return fail(VGX_EHIP, std::string("decode graph: instantiate: ") + hipGetErrorString(ei));
        }
        *graph = g;
        *exec = x;
        return VGX_OK;
    }

    // Caches and buffers for nseq sequences in lockstep (kept for later calls
    // with as many or fewer).
    int ensure_batch(int nseq, size_t ntok) {
        int st;
        if (conv) return fail(VGX_EINVAL, "batched decode: conv (hybrid) models are not supported");
        if (nseq > pcap) return fail(VGX_EINVAL, "batched decode: more than " + std::to_string(pcap) + " sequences");
        if (!head_cat && (st = vgx_mat_concat(ctx, (int)head_tiles.size(), head_tiles.data(), &head_cat))) return st;
        if (nseq > nseq_b) {
            vgx_attn_free(attn_b);
            attn_b = nullptr;
            nseq_b = 0;
            if ((st = vgx_attn_create_seqs(ctx, &attn_desc, nseq, &attn_b))) return st;
            if ((st = dalloc(&blog, (size_t)nseq * m.vocab))) return st;
            nseq_b = nseq;
        }
        if (ntok > btok_cap) {
            if ((st = dalloc(&btok, ntok))) return st;
            btok_cap = ntok;
        }
        return VGX_OK;
    }

    // One position of nseq sequences at once: forward() on each row, the
    // GEMVs as GEMMs over the nseq rows, the attention of every sequence on
    // its own cache in one launch, the final norm + LM head + argmax per row.
    int forward_seqs(const int* toks_dev, int pos, int nseq, int* next_dev) {
        int st;
        const int D = m.dim;
        const float eps = m.rms_eps;
        // the embedding rows with the first attention norm; every later norm
        // comes out of the GEMM that writes the residual stream (wo: the FFN
        // norm; w2: the next layer's attention norm, or the final norm after
        // the last layer), so qkv, the gate and the head read normalised rows
        if ((st = vgx_embed_q8_rms_batch(ctx, emb, emb_scale, m.vocab, D, nseq, toks_dev, bh, L[0].rms_att, eps, bxn)))
            return st;
        for (int l = 0; l < m.layers; ++l) {
            Layer& ly = L[l];
            const int16_t* next_norm = l + 1 < m.layers ? L[l + 1].rms_att : rms_final;
            if ((st = vgx_gemm(ctx, ly.qkv, nseq, bxn, nullptr, bqkv))) return st;
            if ((st = vgx_attn_block_seqs(attn_b, l, pos, nseq, bqkv, batt))) return st;
            if ((st = vgx_gemm_norm(ctx, ly.wo, nseq, batt, bh, bx1, ly.rms_ffn, eps, bxn))) return st;
            if ((st = vgx_ffn_gate_batch(ctx, ly.w1, ly.w3, nseq, bxn, ly.hs, bhid))) return st;
            if (ffn_chunk)
                st = vgx_gemm_add_split_norm(ctx, ly.w2, ffn_chunk, nseq, bhid, bx1, bh, next_norm, eps, bxn);
            else
                st = vgx_gemm_norm(ctx, ly.w2, nseq, bhid, bx1, bh, next_norm, eps, bxn);
            if (st) return st;
        }
        if ((st = vgx_gemm(ctx, head_cat, nseq, bxn, nullptr, blog))) return st;
        return vgx_argmax_rows(ctx, nseq, m.vocab, blog, next_dev);
    }
};

extern "C" {

static int engine_finish_open(vgx_engine* e, int device, int seq, int kv_bits, vgx_engine** out) {
    g_err.clear();
    int st = e->init(device, seq, kv_bits);
    if (st) {
        std::string msg = g_err.empty() ? vgx_last_error() : g_err;
        delete e;
        g_err = msg;
        return st;
    }
    *out = e;
    return VGX_OK;
}

int vgx_engine_open(const char* path, int device, int seq, int kv_bits, vgx_engine** out) {
    if (!path || !out) return fail(VGX_EINVAL, "vgx_engine_open: NULL argument");
    *out = nullptr;
    vgx_engine* e = new vgx_engine();
    std::string err;
    if (!e->c.open(path, err)) { delete e; return fail(VGX_EINVAL, err); }
    struct stat st {};
    if (stat(path, &st) == 0) {
        e->src_size = (uint64_t)st.st_size;
        e->src_mtime = (uint64_t)st.st_mtime;
    }
    return engine_finish_open(e, device, seq, kv_bits, out);
}

int vgx_engine_open_bytes(const void* data, size_t size, int device, int seq, int kv_bits, vgx_engine** out) {
    if (!data || !out) return fail(VGX_EINVAL, "vgx_engine_open_bytes: NULL argument");
    *out = nullptr;
    vgx_engine* e = new vgx_engine();
    std::string err;
    if (!e->c.open_bytes(static_cast<const uint8_t*>(data), size, err)) { delete e; return fail(VGX_EINVAL, err); }
    e->src_size = size;  // no file: mtime 0
    return engine_finish_open(e, device, seq, kv_bits, out);
}

int vgx_engine_close(vgx_engine* e) {
    delete e;
    return VGX_OK;
}

int vgx_engine_info(const vgx_engine* e, int* dim, int* layers, int* vocab, int* seq) {
    if (!e) return fail(VGX_EINVAL, "vgx_engine_info: NULL engine");
    if (dim) *dim = e->m.dim;
    if (layers) *layers = e->m.layers;
    if (vocab) *vocab = e->m.vocab;
    if (seq) *seq = e->seq;
    return VGX_OK;
}

int vgx_engine_conv_layers(const vgx_engine* e) {
    if (!e) return -1;
    int n = 0;
    for (int l = 0; l < e->m.layers; ++l) n += e->is_conv(l) ? 1 : 0;
    return n;
}

int vgx_engine_step(vgx_engine* e, int token, int pos, int16_t* logits_host, int* next) {
    g_err.clear();
    if (!e) return fail(VGX_EINVAL, "vgx_engine_step: NULL engine");
    if (pos < 0 || pos >= e->seq) return fail(VGX_ERANGE, "vgx_engine_step: position outside the KV length");
    if (token < 0 || token >= e->m.vocab) return fail(VGX_EINVAL, "vgx_engine_step: token outside the vocabulary");
    hipStream_t s = static_cast<hipStream_t>(vgx_ctx_stream(e->ctx));
    int* slot = e->toks + e->seq;
    if (hipMemcpyAsync(slot, &token, sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess)
        return fail(VGX_EHIP, "token upload");
    int st = e->forward(slot, pos, true, slot, e->attn);
    if (st) return st;
    if (logits_host && hipMemcpyAsync(logits_host, e->logits, (size_t)e->m.vocab * 2, hipMemcpyDeviceToHost, s) != hipSuccess)
        return fail(VGX_EHIP, "logits readback");
    int nx = 0;
    if (hipMemcpyAsync(&nx, slot, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess) return fail(VGX_EHIP, "token readback");
    if (hipStreamSynchronize(s) != hipSuccess) return fail(VGX_EHIP, "step sync");
    if (next) *next = nx;
    return VGX_OK;
}

int vgx_engine_step_candidates(vgx_engine* e, int token, int pos, int topk, float temp, float top_p, float* value,
                               int* cand_token, int cap, int* n, float* stats, int* complete, float* full) {
    g_err.clear();
    if (!e || !value || !cand_token || !n || !stats || !complete || !full)
        return fail(VGX_EINVAL, "vgx_engine_step_candidates: NULL argument");
    if (topk <= 0 || cap < topk) return fail(VGX_EINVAL, "vgx_engine_step_candidates: need 0 < top_k <= cap");
    if (!e->cand_tiles_ok)
        return fail(VGX_EINVAL, "vgx_engine_step_candidates: an LM-head tile before the last is not a multiple of 16 rows");
    if (pos < 0 || pos >= e->seq) return fail(VGX_ERANGE, "vgx_engine_step_candidates: position outside the KV length");
    if (token < 0 || token >= e->m.vocab)
        return fail(VGX_EINVAL, "vgx_engine_step_candidates: token outside the vocabulary");
    const int V = e->m.vocab, nch = (V + 15) / 16;
    int st;
    if (!e->chunk_dev && (st = e->dalloc(&e->chunk_dev, (size_t)nch * 6))) return st;
    e->chunk_host.resize((size_t)nch * 6);
    hipStream_t s = static_cast<hipStream_t>(vgx_ctx_stream(e->ctx));
    int* slot = e->toks + e->seq;
    if (hipMemcpyAsync(slot, &token, sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess)
        return fail(VGX_EHIP, "token upload");
    if ((st = e->forward(slot, pos, true, slot, e->attn))) return st;
    if ((st = vgx_logits_chunks(e->ctx, e->logits, V, temp, e->chunk_dev))) return st;
    if (hipMemcpyAsync(e->chunk_host.data(), e->chunk_dev, (size_t)nch * 6 * sizeof(int), hipMemcpyDeviceToHost, s) !=
            hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return fail(VGX_EHIP, "candidate readback");
    // GPU::logits_candidates_from's host side (engine/src/gpu_matvec.cpp:
    // 175-229): both ranks of every chunk are candidates, in chunk order,
    // then sorted by value; the softmax denominator comes from the chunks'
    // (max, sum) pairs rescaled to the global maximum; the top_k kept
    // candidates are complete when their probability reaches top_p.
    struct Cand {
        float value;
        int token;
    };
    std::vector<Cand> cand;
    cand.reserve((size_t)nch * 2);
    std::vector<float> cmax((size_t)nch, -1e30f), csum((size_t)nch, 0.0f);
    float gmax = -1e30f;
    for (int g = 0; g < nch; ++g) {
        const int* o = &e->chunk_host[(size_t)g * 6];
        for (int r = 0; r < 2; ++r) {
            if (o[2 * r + 1] < 0) continue;  // a one-logit chunk has no second
            const float v = (float)o[2 * r] / 256.0f;
            cand.push_back(Cand{v, o[2 * r + 1]});
            cmax[(size_t)g] = std::max(cmax[(size_t)g], v);
            gmax = std::max(gmax, v);
        }
        const float mx = (float)o[4] / 256.0f;
        cmax[(size_t)g] = std::max(cmax[(size_t)g], mx);
        csum[(size_t)g] = (float)o[5] / 2048.0f;
        gmax = std::max(gmax, mx);
    }
    std::sort(cand.begin(), cand.end(), [](const Cand& a, const Cand& b) { return a.value > b.value; });
    const float T = std::max(0.0001f, temp);
    float denom = 0.0f;
    for (int g = 0; g < nch; ++g) denom += csum[(size_t)g] * expf((cmax[(size_t)g] - gmax) / T);
    if ((int)cand.size() > topk) cand.resize((size_t)topk);
    float cum = 0.0f;
    for (const Cand& c : cand) cum += expf((c.value - gmax) / T) / denom;
    for (size_t i = 0; i < cand.size(); ++i) {
        value[i] = cand[i].value;
        cand_token[i] = cand[i].token;
    }
    *n = (int)cand.size();
    stats[0] = logf(denom) + gmax / T;  // logsumexp of v / T
    stats[1] = gmax;
    stats[2] = denom;
    *complete = cum + 1e-6f >= top_p ? 1 : 0;
    if (!*complete) {
        // the reference falls back to the full read-back of the same pass
        e->logits_tmp.resize((size_t)V);
        if (hipMemcpy(e->logits_tmp.data(), e->logits, (size_t)V * 2, hipMemcpyDeviceToHost) != hipSuccess)
            return fail(VGX_EHIP, "logits readback");
        for (int i = 0; i < V; ++i) full[i] = (float)e->logits_tmp[(size_t)i] / 256.0f;
    }
    return VGX_OK;
}

int vgx_engine_generate(vgx_engine* e, const int* prompt, int n_prompt, int n_gen, int* out,
                        double* prefill_ms, double* decode_ms) {
    return vgx_engine_generate_from(e, prompt, n_prompt, 0, n_gen, out, prefill_ms, decode_ms);
}

int vgx_engine_generate_from(vgx_engine* e, const int* prompt, int n_prompt, int n_cached, int n_gen, int* out,
                             double* prefill_ms, double* decode_ms) {
    g_err.clear();
    if (!e || !prompt || !out) return fail(VGX_EINVAL, "vgx_engine_generate: NULL argument");
    if (n_prompt <= 0 || n_gen <= 0 || n_prompt + n_gen - 1 > e->seq)
        return fail(VGX_ERANGE, "vgx_engine_generate: prompt + generation longer than the KV length");
    if (n_cached < 0 || n_cached >= n_prompt)
        return fail(VGX_ERANGE, "vgx_engine_generate: the cached prefix must leave at least one prompt token");
    for (int i = 0; i < n_prompt; ++i)
        if (prompt[i] < 0 || prompt[i] >= e->m.vocab) return fail(VGX_EINVAL, "prompt token outside the vocabulary");
    hipStream_t s = static_cast<hipStream_t>(vgx_ctx_stream(e->ctx));
    // history: toks[0..n_prompt) the prompt, then the generated tokens
    int* gen = e->toks + n_prompt;
    if (hipMemcpy(e->toks, prompt, (size_t)n_prompt * sizeof(int), hipMemcpyHostToDevice) != hipSuccess)
        return fail(VGX_EHIP, "prompt upload");
    if (hipDeviceSynchronize() != hipSuccess) return fail(VGX_EHIP, "sync");
    auto t0 = std::chrono::steady_clock::now();
    int st;
    if ((st = e->run_prompt(e->toks + n_cached, n_cached, n_prompt - n_cached, gen, e->attn))) return st;
    if (hipStreamSynchronize(s) != hipSuccess) return fail(VGX_EHIP, "prefill sync");
    auto t1 = std::chrono::steady_clock::now();
    if (e->use_graph && n_gen > 1) {
        // the step graph from position n_prompt: tok_cur = gen[0], pos = n_prompt
        if ((st = e->ensure_step_graph())) return st;
        e->pos_host = n_prompt;  // the copy's source outlives the call's queueing
        if (hipMemcpyAsync(e->tok_cur, gen, sizeof(int), hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipMemcpyAsync(e->pos_dev, &e->pos_host, sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess)
            return fail(VGX_EHIP, "decode graph: state upload");
        // the first replay's input; each replay embeds the next one's
        if ((st = vgx_embed_q8(e->ctx, e->emb, e->emb_scale, e->m.vocab, e->m.dim, e->tok_cur, e->h))) return st;
        // tokens i .. i + kMultiSteps - 1 per multi-step replay, the rest one a replay
        int i = 1;
        if (e->multi_exec)
            for (; i + vgx_engine::kMultiSteps <= n_gen; i += vgx_engine::kMultiSteps)
                if (hipGraphLaunch(e->multi_exec, s) != hipSuccess) return fail(VGX_EHIP, "decode graph: launch");
        for (; i < n_gen; ++i)
            if (hipGraphLaunch(e->step_exec, s) != hipSuccess) return fail(VGX_EHIP, "decode graph: launch");
    } else {
        for (int i = 1; i < n_gen; ++i)
            if ((st = e->forward(gen + i - 1, n_prompt + i - 1, true, gen + i, e->attn))) return st;
    }
    if (hipStreamSynchronize(s) != hipSuccess) return fail(VGX_EHIP, "decode sync");
    auto t2 = std::chrono::steady_clock::now();
    if (hipMemcpy(out, gen, (size_t)n_gen * sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
        return fail(VGX_EHIP, "token readback");
    if (prefill_ms) *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (decode_ms) *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    return VGX_OK;
}

int vgx_engine_set_graphs(vgx_engine* e, int on) {
    g_err.clear();
    if (!e) return fail(VGX_EINVAL, "vgx_engine_set_graphs: NULL engine");
    e->use_graph = on != 0;
    return VGX_OK;
}

int vgx_engine_set_prefill_batch(vgx_engine* e, int n) {
    g_err.clear();
    if (!e) return fail(VGX_EINVAL, "vgx_engine_set_prefill_batch: NULL engine");
    if (n < 0 || n > e->pcap)
        return fail(VGX_EINVAL, "vgx_engine_set_prefill_batch: batch outside 0.." + std::to_string(e->pcap));
    e->pbatch = n;
    return VGX_OK;
}

int vgx_engine_prefill(vgx_engine* e, const int* tokens, int n, int pos0, int16_t* logits_host, int* next) {
    g_err.clear();
    if (!e || !tokens) return fail(VGX_EINVAL, "vgx_engine_prefill: NULL argument");
    if (n <= 0 || pos0 < 0 || pos0 > e->seq - n)
        return fail(VGX_ERANGE, "vgx_engine_prefill: positions outside the KV length");
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= e->m.vocab) return fail(VGX_EINVAL, "vgx_engine_prefill: token outside the vocabulary");
    hipStream_t s = static_cast<hipStream_t>(vgx_ctx_stream(e->ctx));
    int* dst = e->toks + pos0;
    int* slot = e->toks + e->seq;
    if (hipMemcpyAsync(dst, tokens, (size_t)n * sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess)
        return fail(VGX_EHIP, "token upload");
    int st = e->run_prompt(dst, pos0, n, slot, e->attn);
    if (st) return st;
    if (logits_host && hipMemcpyAsync(logits_host, e->logits, (size_t)e->m.vocab * 2, hipMemcpyDeviceToHost, s) != hipSuccess)
        return fail(VGX_EHIP, "logits readback");
    int nx = 0;
    if (hipMemcpyAsync(&nx, slot, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess) return fail(VGX_EHIP, "token readback");
    if (hipStreamSynchronize(s) != hipSuccess) return fail(VGX_EHIP, "prefill sync");
    if (next) *next = nx;
    return VGX_OK;
}

int vgx_engine_generate_batch(vgx_engine* e, int nseq, const int* prompts, int n_prompt, int n_gen, int* out,
                              double* prefill_ms, double* decode_ms) {
    g_err.clear();
    if (!e || !prompts || !out) return fail(VGX_EINVAL, "vgx_engine_generate_batch: NULL argument");
    if (nseq <= 0) return fail(VGX_EINVAL, "vgx_engine_generate_batch: nseq <= 0");
    if (n_prompt <= 0 || n_gen <= 0 || n_prompt + n_gen - 1 > e->seq)
        return fail(VGX_ERANGE, "vgx_engine_generate_batch: prompt + generation longer than the KV length");
    const size_t np = (size_t)nseq * n_prompt, ng = (size_t)nseq * n_gen;
    for (size_t i = 0; i < np; ++i)
        if (prompts[i] < 0 || prompts[i] >= e->m.vocab) return fail(VGX_EINVAL, "prompt token outside the vocabulary");
    int st;
    if ((st = e->ensure_batch(nseq, np + ng))) return st;
    hipStream_t s = static_cast<hipStream_t>(vgx_ctx_stream(e->ctx));
    // device tokens: the prompts [nseq][n_prompt], then the generated tokens
    // step-major [n_gen][nseq] (one step's tokens are the next step's input)
    int* dprompt = e->btok;
    int* gen = e->btok + np;
    if (hipMemcpy(dprompt, prompts, np * sizeof(int), hipMemcpyHostToDevice) != hipSuccess)
        return fail(VGX_EHIP, "prompt upload");
    if (hipDeviceSynchronize() != hipSuccess) return fail(VGX_EHIP, "sync");
    auto t0 = std::chrono::steady_clock::now();
    for (int q = 0; q < nseq; ++q) {
        vgx_attn* view = nullptr;
        if ((st = vgx_attn_seq_view(e->attn_b, q, &view))) return st;
        st = e->run_prompt(dprompt + (size_t)q * n_prompt, 0, n_prompt, gen + q, view);
        vgx_attn_free(view);
        if (st) return st;
    }
    if (hipStreamSynchronize(s) != hipSuccess) return fail(VGX_EHIP, "prefill sync");
    auto t1 = std::chrono::steady_clock::now();
    for (int i = 1; i < n_gen; ++i)
        if ((st = e->forward_seqs(gen + (size_t)(i - 1) * nseq, n_prompt + i - 1, nseq, gen + (size_t)i * nseq)))
            return st;
    if (hipStreamSynchronize(s) != hipSuccess) return fail(VGX_EHIP, "decode sync");
    auto t2 = std::chrono::steady_clock::now();
    std::vector<int> g(ng);
    if (hipMemcpy(g.data(), gen, ng * sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
        return fail(VGX_EHIP, "token readback");
    for (int q = 0; q < nseq; ++q)
        for (int i = 0; i < n_gen; ++i) out[(size_t)q * n_gen + i] = g[(size_t)i * nseq + q];
    if (prefill_ms) *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (decode_ms) *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    return VGX_OK;
}

// ---------------------------------------------------------------------------
// The MMKV1 prefix cache (engine/src/prefix_cache.cpp:25-207): a header that
// names the container (size, mtime), the shape and the KV packing, the token
// ids, then per layer the n KV rows in the texel byte layout (q16 big-endian,
// q8 bytes), and for a hybrid (version 4) the two conv history rows of every
// conv layer (x[pos-2], then x[pos-1]; q16 big-endian, two per texel).  A
// conv layer has no KV cache; its row block is written as zeros and skipped
// on load.  The JSON sidecar (path + ".json") repeats the header's fields.

namespace {

struct MmkvHeader {
    uint32_t version, dim, hidden, layers, heads, kv_heads, vocab, seq, head_dim, flags, n, width, vsw;
    uint64_t size, mtime;
    float theta, kscale;
};

MmkvHeader mmkv_expect(const vgx_engine* e, uint32_t n) {
    MmkvHeader h{};
    const bool hybrid = e->conv != nullptr;
    h.version = hybrid ? 4u : 2u;
    h.size = e->src_size;
    h.mtime = e->src_mtime;
    h.dim = (uint32_t)e->m.dim;
    h.hidden = (uint32_t)e->m.hidden;
    h.layers = (uint32_t)e->m.layers;
    h.heads = (uint32_t)e->m.heads;
    h.kv_heads = (uint32_t)e->m.kv_heads;
    h.vocab = (uint32_t)e->m.vocab;
    h.seq = (uint32_t)e->seq;
    h.head_dim = (uint32_t)e->m.head_dim();
    h.theta = e->m.theta;
    // qk_norm 1, rope_half 2, KV q16 4 / q8 8, 8-bit activations 16, hybrid 32
    h.flags = (e->m.qk_norm ? 1u : 0u) | (e->m.rope_half ? 2u : 0u) | (e->kv_bits == 16 ? 4u : 8u) |
              (hybrid ? 32u : 0u);
    h.n = n;
    const int kv_dim = e->m.kv_dim();
    h.width = (uint32_t)(e->kv_bits == 16 ? kv_dim : kv_dim / 2);  // texels per KV row
    h.vsw = 0;
    h.kscale = e->kv_bits == 16 ? 2048.0f : 16.0f;
    return h;
}

std::string hex64(uint64_t v) {
    char b[32];
    std::snprintf(b, sizeof(b), "%016llx", (unsigned long long)v);
    return b;
}

}  // namespace

int vgx_engine_save_prefix(vgx_engine* e, const char* path, const int* toks, int n, uint64_t system_fnv,
                           uint64_t tools_fnv) {
    g_err.clear();
    if (!e || !path || !toks) return fail(VGX_EINVAL, "vgx_engine_save_prefix: NULL argument");
    if (n <= 0 || n > e->seq) return fail(VGX_ERANGE, "vgx_engine_save_prefix: token count outside 1..seq");
    const MmkvHeader h = mmkv_expect(e, (uint32_t)n);
    std::ofstream f(path, std::ios::binary);
    if (!f) return fail(VGX_EINVAL, std::string("vgx_engine_save_prefix: cannot write ") + path);
    const char magic[8] = {'M', 'M', 'K', 'V', '1', 0, 0, 0};
    f.write(magic, 8);
    auto u32 = [&](uint32_t v) { f.write(reinterpret_cast<const char*>(&v), 4); };
    auto u64 = [&](uint64_t v) { f.write(reinterpret_cast<const char*>(&v), 8); };
    auto f32 = [&](float v) { f.write(reinterpret_cast<const char*>(&v), 4); };
    u32(h.version);
    u64(h.size);
    u64(h.mtime);
    u32(h.dim); u32(h.hidden); u32(h.layers); u32(h.heads);
    u32(h.kv_heads); u32(h.vocab); u32(h.seq); u32(h.head_dim);
    f32(h.theta);
    u32(h.flags);
    u32(h.n);
    u32(h.width);
    if (h.version >= 3) u32(h.vsw);
    f32(h.kscale);
    uint64_t fnv = 1469598103934665603ull;  // FNV-1a over the ids' little-endian bytes
    for (int i = 0; i < n; ++i) {
        u32((uint32_t)toks[i]);
        for (int b = 0; b < 4; ++b) {
            fnv ^= (uint8_t)((uint32_t)toks[i] >> (8 * b));
            fnv *= 1099511628211ull;
        }
    }
    const int rb = vgx_kv_row_bytes(e->attn);
    std::vector<uint8_t> rows((size_t)rb * n);
    for (int l = 0; l < e->m.layers; ++l) {
        if (e->is_conv(l)) {
            std::fill(rows.begin(), rows.end(), 0);
        } else {
            int st = vgx_kv_read_rows(e->attn, l, 0, n, rows.data());
            if (st) return st;
        }
        f.write(reinterpret_cast<const char*>(rows.data()), (std::streamsize)rows.size());
    }
    if (e->conv) {
        const int D = e->m.dim;
        std::vector<int16_t> st2((size_t)2 * D);
        std::vector<uint8_t> be((size_t)2 * D);
        for (int l = 0; l < e->m.layers; ++l) {
            if (!e->is_conv(l)) continue;
            int st = vgx_conv_state_read(e->conv, l, st2.data());
            if (st) return st;
            for (int which = 0; which < 2; ++which) {
                for (int i = 0; i < D; ++i) {
                    const uint16_t v = (uint16_t)st2[(size_t)which * D + i];
                    be[2 * i] = (uint8_t)(v >> 8);
                    be[2 * i + 1] = (uint8_t)(v & 0xFF);
                }
                f.write(reinterpret_cast<const char*>(be.data()), (std::streamsize)be.size());
            }
        }
    }
    if (!f) return fail(VGX_EHIP, std::string("vgx_engine_save_prefix: write failed: ") + path);
    f.close();
    std::ofstream sm(std::string(path) + ".json");
    if (sm) {
        sm << "{\"format\":\"mmkv\",\"version\":" << h.version << ",\"source_size\":" << h.size
           << ",\"source_mtime\":" << h.mtime << ",\"dim\":" << h.dim << ",\"hidden\":" << h.hidden
           << ",\"layers\":" << h.layers << ",\"heads\":" << h.heads << ",\"kv_heads\":" << h.kv_heads
           << ",\"vocab\":" << h.vocab << ",\"seq\":" << h.seq << ",\"head_dim\":" << h.head_dim
           << ",\"rope_theta\":" << (double)h.theta << ",\"kv_bits\":" << e->kv_bits << ",\"act_fmt\":\"x16_2\""
           << ",\"hybrid\":" << (e->conv ? "true" : "false") << ",\"kv_scale\":" << (double)h.kscale
           << ",\"kv_width\":" << h.width << ",\"vstep\":0,\"n_tokens\":" << n << ",\"tokens_fnv64\":\""
           << hex64(fnv) << "\",\"system_fnv64\":\"" << hex64(system_fnv) << "\",\"tools_fnv64\":\""
           << hex64(tools_fnv) << "\",\"template\":\"\"}\n";
    }
    return VGX_OK;
}

int vgx_engine_load_prefix(vgx_engine* e, const char* path, int* toks, int cap, int* n_out) {
    g_err.clear();
    if (!e || !path || !n_out) return fail(VGX_EINVAL, "vgx_engine_load_prefix: NULL argument");
    *n_out = 0;
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail(VGX_EINVAL, std::string("vgx_engine_load_prefix: cannot read ") + path);
    char magic[8] = {};
    f.read(magic, 8);
    if (!f || std::memcmp(magic, "MMKV1", 5) != 0) return fail(VGX_EINVAL, "vgx_engine_load_prefix: not an MMKV1 file");
    MmkvHeader h{};
    auto u32 = [&](uint32_t& v) { f.read(reinterpret_cast<char*>(&v), 4); };
    auto u64 = [&](uint64_t& v) { f.read(reinterpret_cast<char*>(&v), 8); };
    u32(h.version);
    u64(h.size);
    u64(h.mtime);
    u32(h.dim); u32(h.hidden); u32(h.layers); u32(h.heads);
    u32(h.kv_heads); u32(h.vocab); u32(h.seq); u32(h.head_dim);
    f.read(reinterpret_cast<char*>(&h.theta), 4);
    u32(h.flags);
    u32(h.n);
    u32(h.width);
    if (h.version >= 3) u32(h.vsw);
    f.read(reinterpret_cast<char*>(&h.kscale), 4);
    const MmkvHeader w = mmkv_expect(e, h.n);
    // load_prefix_cache's refusals (engine/src/prefix_cache.cpp:151-168): a
    // cache for another container, shape or packing is not loaded
    if (!f || h.version != w.version || h.size != w.size || h.mtime != w.mtime || h.dim != w.dim ||
        h.hidden != w.hidden || h.layers != w.layers || h.heads != w.heads || h.kv_heads != w.kv_heads ||
        h.vocab != w.vocab || h.seq != w.seq || h.head_dim != w.head_dim || h.theta != w.theta ||
        h.flags != w.flags || h.width != w.width || h.vsw != 0 || h.n == 0 || h.n > (uint32_t)e->seq ||
        std::memcmp(&h.kscale, &w.kscale, 4) != 0)
        return fail(VGX_EINVAL, "vgx_engine_load_prefix: the cache was written for another model, shape or KV packing");
    if (toks && (int)h.n > cap) return fail(VGX_ERANGE, "vgx_engine_load_prefix: token buffer too small");
    std::vector<int> ids(h.n);
    for (uint32_t i = 0; i < h.n; ++i) {
        uint32_t v = 0;
        u32(v);
        ids[i] = (int)v;
    }
    const int rb = vgx_kv_row_bytes(e->attn);
    std::vector<uint8_t> rows((size_t)rb * h.n);
    std::vector<std::vector<uint8_t>> kv((size_t)e->m.layers);
    for (int l = 0; l < e->m.layers; ++l) {
        f.read(reinterpret_cast<char*>(rows.data()), (std::streamsize)rows.size());
        if (!f) return fail(VGX_EINVAL, "vgx_engine_load_prefix: truncated KV rows");
        if (!e->is_conv(l)) kv[l] = rows;
    }
    std::vector<std::vector<int16_t>> cs;
    if (e->conv) {
        const int D = e->m.dim;
        std::vector<uint8_t> be((size_t)2 * D);
        cs.assign((size_t)e->m.layers, {});
        for (int l = 0; l < e->m.layers; ++l) {
            if (!e->is_conv(l)) continue;
            cs[l].resize((size_t)2 * D);
            for (int which = 0; which < 2; ++which) {
                f.read(reinterpret_cast<char*>(be.data()), (std::streamsize)be.size());
                if (!f) return fail(VGX_EINVAL, "vgx_engine_load_prefix: truncated conv history");
                for (int i = 0; i < D; ++i)
                    cs[l][(size_t)which * D + i] = (int16_t)(uint16_t)((be[2 * i] << 8) | be[2 * i + 1]);
            }
        }
    }
    // everything read and checked: now the device state changes
    int st;
    for (int l = 0; l < e->m.layers; ++l)
        if (!e->is_conv(l) && (st = vgx_kv_write_rows(e->attn, l, 0, (int)h.n, kv[l].data()))) return st;
    for (int l = 0; e->conv && l < e->m.layers; ++l)
        if (e->is_conv(l) && (st = vgx_conv_state_write(e->conv, l, cs[l].data()))) return st;
    if (hipMemcpy(e->toks, ids.data(), (size_t)h.n * sizeof(int), hipMemcpyHostToDevice) != hipSuccess)
        return fail(VGX_EHIP, "token history upload");
    if (toks) std::memcpy(toks, ids.data(), (size_t)h.n * sizeof(int));
    *n_out = (int)h.n;
    return VGX_OK;
}

const char* vgx_engine_last_error(void) { return g_err.empty() ? vgx_last_error() : g_err.c_str(); }

}  // extern "C"
