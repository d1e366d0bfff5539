/*
 * CPU oracle of the speech-tokenizer decoder.  TEST INFRASTRUCTURE ONLY (see
 * codec_oracle.h).  CS = native/qwen3-tts-native-codec/native/src/codec_state.cu.
 *
 * Pipeline of one packet of F frames (CS:3989-4089):
 *   RVQ (16 codebooks) -> 512-d, causal pre-convolution k=3 -> 1024-d
 *   8-layer transformer, one frame at a time (hidden 512, 16 heads of 64,
 *     72-position sliding KV window) -> 1024-d
 *   2 x (transposed conv x2 + ConvNeXt block) -> 4F latent positions
 *   causal conv k=7 1024 -> 1536, 4 x (SnakeBeta, transposed conv with
 *     stride 8 / 5 / 4 / 3, 3 residual units with dilations 1, 3, 9),
 *   SnakeBeta, causal conv k=7 96 -> 1, clamp, 16-bit PCM.
 */
#include "codec_oracle.h"

#include "oracle.h"
#include "../qwen3-tts-native_amd/csrc/q3_math.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum {
    KV_WINDOW = 72,
    HEADS = 16,
    HEAD_DIM = 64,
    LAYERS = 8,
    HIDDEN = 512,
    MAX_FRAMES = 4,
};

/* ---- tensor table ------------------------------------------------------ */
enum {
    T_RVQ_FIRST_EMB = 0,
    T_RVQ_FIRST_USAGE = 1,
    T_RVQ_REST_EMB = 2,     /* + codebook - 1, 15 of them */
    T_RVQ_REST_USAGE = 17,  /* + codebook - 1 */
    T_RVQ_FIRST_PROJ = 32,
    T_RVQ_REST_PROJ = 33,
    T_PRECONV_W = 34,
    T_PRECONV_B = 35,
    T_INPUT_PROJ_W = 36,
    T_INPUT_PROJ_B = 37,
    T_LAYER = 38, /* + 11 * layer + one of L_* */
    T_NORM = 126,
    T_OUTPUT_PROJ_W = 127,
    T_OUTPUT_PROJ_B = 128,
    T_UPSAMPLE = 129, /* + 11 * stage + one of U_* */
    T_DEC0_W = 151,
    T_DEC0_B = 152,
    T_STAGE = 153, /* + 28 * stage + one of S_* (+ 8 * unit for units) */
    T_DEC5_ALPHA = 265,
    T_DEC5_BETA = 266,
    T_DEC6_W = 267,
    T_DEC6_B = 268,
};
enum { L_IN_NORM, L_Q, L_K, L_V, L_O, L_ATTN_SCALE, L_POST_NORM, L_GATE, L_UP, L_DOWN, L_MLP_SCALE };
enum { U_CONV_W, U_CONV_B, U_DW_W, U_DW_B, U_NORM_W, U_NORM_B, U_PW1_W, U_PW1_B, U_PW2_W, U_PW2_B, U_GAMMA };
enum { S_ALPHA, S_BETA, S_TCONV_W, S_TCONV_B, S_UNIT };
enum { R_ACT1_ALPHA, R_ACT1_BETA, R_CONV1_W, R_CONV1_B, R_ACT2_ALPHA, R_ACT2_BETA, R_CONV2_W, R_CONV2_B };

static const int kStageIn[4] = {1536, 768, 384, 192};
static const int kStageOut[4] = {768, 384, 192, 96};
static const int kStride[4] = {8, 5, 4, 3};
static const int kDilation[3] = {1, 3, 9};

static char g_names[ORC_CODEC_TENSORS][96];
static uint64_t g_elements[ORC_CODEC_TENSORS];
static int g_table_ready = 0;

static void set(int i, uint64_t elements, const char* name) {
    snprintf(g_names[i], sizeof(g_names[i]), "%s", name);
    g_elements[i] = elements;
}

static void build_table(void) {
    char n[96];
    if (g_table_ready) return;
    set(T_RVQ_FIRST_EMB, 2048ull * 256, "decoder.quantizer.rvq_first.vq.layers.0._codebook.embedding_sum");
    set(T_RVQ_FIRST_USAGE, 2048, "decoder.quantizer.rvq_first.vq.layers.0._codebook.cluster_usage");
    for (int c = 0; c < 15; ++c) {
        snprintf(n, sizeof(n), "decoder.quantizer.rvq_rest.vq.layers.%d._codebook.embedding_sum", c);
        set(T_RVQ_REST_EMB + c, 2048ull * 256, n);
        snprintf(n, sizeof(n), "decoder.quantizer.rvq_rest.vq.layers.%d._codebook.cluster_usage", c);
        set(T_RVQ_REST_USAGE + c, 2048, n);
    }
    set(T_RVQ_FIRST_PROJ, 512ull * 256, "decoder.quantizer.rvq_first.output_proj.weight");
    set(T_RVQ_REST_PROJ, 512ull * 256, "decoder.quantizer.rvq_rest.output_proj.weight");
    set(T_PRECONV_W, 1024ull * 512 * 3, "decoder.pre_conv.conv.weight");
    set(T_PRECONV_B, 1024, "decoder.pre_conv.conv.bias");
    set(T_INPUT_PROJ_W, 512ull * 1024, "decoder.pre_transformer.input_proj.weight");
    set(T_INPUT_PROJ_B, 512, "decoder.pre_transformer.input_proj.bias");
    for (int l = 0; l < LAYERS; ++l) {
        const int b = T_LAYER + 11 * l;
        const char* p = "decoder.pre_transformer.layers";
        snprintf(n, sizeof(n), "%s.%d.input_layernorm.weight", p, l); set(b + L_IN_NORM, 512, n);
        snprintf(n, sizeof(n), "%s.%d.self_attn.q_proj.weight", p, l); set(b + L_Q, 1024ull * 512, n);
        snprintf(n, sizeof(n), "%s.%d.self_attn.k_proj.weight", p, l); set(b + L_K, 1024ull * 512, n);
        snprintf(n, sizeof(n), "%s.%d.self_attn.v_proj.weight", p, l); set(b + L_V, 1024ull * 512, n);
        snprintf(n, sizeof(n), "%s.%d.self_attn.o_proj.weight", p, l); set(b + L_O, 512ull * 1024, n);
        snprintf(n, sizeof(n), "%s.%d.self_attn_layer_scale.scale", p, l); set(b + L_ATTN_SCALE, 512, n);
        snprintf(n, sizeof(n), "%s.%d.post_attention_layernorm.weight", p, l); set(b + L_POST_NORM, 512, n);
        snprintf(n, sizeof(n), "%s.%d.mlp.gate_proj.weight", p, l); set(b + L_GATE, 1024ull * 512, n);
        snprintf(n, sizeof(n), "%s.%d.mlp.up_proj.weight", p, l); set(b + L_UP, 1024ull * 512, n);
        snprintf(n, sizeof(n), "%s.%d.mlp.down_proj.weight", p, l); set(b + L_DOWN, 512ull * 1024, n);
        snprintf(n, sizeof(n), "%s.%d.mlp_layer_scale.scale", p, l); set(b + L_MLP_SCALE, 512, n);
    }
    set(T_NORM, 512, "decoder.pre_transformer.norm.weight");
    set(T_OUTPUT_PROJ_W, 1024ull * 512, "decoder.pre_transformer.output_proj.weight");
    set(T_OUTPUT_PROJ_B, 1024, "decoder.pre_transformer.output_proj.bias");
    for (int s = 0; s < 2; ++s) {
        const int b = T_UPSAMPLE + 11 * s;
        snprintf(n, sizeof(n), "decoder.upsample.%d.0.conv.weight", s); set(b + U_CONV_W, 1024ull * 1024 * 2, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.0.conv.bias", s); set(b + U_CONV_B, 1024, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.dwconv.conv.weight", s); set(b + U_DW_W, 1024ull * 7, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.dwconv.conv.bias", s); set(b + U_DW_B, 1024, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.norm.weight", s); set(b + U_NORM_W, 1024, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.norm.bias", s); set(b + U_NORM_B, 1024, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.pwconv1.weight", s); set(b + U_PW1_W, 4096ull * 1024, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.pwconv1.bias", s); set(b + U_PW1_B, 4096, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.pwconv2.weight", s); set(b + U_PW2_W, 1024ull * 4096, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.pwconv2.bias", s); set(b + U_PW2_B, 1024, n);
        snprintf(n, sizeof(n), "decoder.upsample.%d.1.gamma", s); set(b + U_GAMMA, 1024, n);
    }
    set(T_DEC0_W, 1536ull * 1024 * 7, "decoder.decoder.0.conv.weight");
    set(T_DEC0_B, 1536, "decoder.decoder.0.conv.bias");
    for (int t = 0; t < 4; ++t) {
        const int b = T_STAGE + 28 * t;
        const uint64_t ci = kStageIn[t], co = kStageOut[t];
        snprintf(n, sizeof(n), "decoder.decoder.%d.block.0.alpha", t + 1); set(b + S_ALPHA, ci, n);
        snprintf(n, sizeof(n), "decoder.decoder.%d.block.0.beta", t + 1); set(b + S_BETA, ci, n);
        snprintf(n, sizeof(n), "decoder.decoder.%d.block.1.conv.weight", t + 1);
        set(b + S_TCONV_W, ci * co * 2 * kStride[t], n);
        snprintf(n, sizeof(n), "decoder.decoder.%d.block.1.conv.bias", t + 1); set(b + S_TCONV_B, co, n);
        for (int u = 0; u < 3; ++u) {
            const int r = b + S_UNIT + 8 * u;
            const char* p = "decoder.decoder";
            snprintf(n, sizeof(n), "%s.%d.block.%d.act1.alpha", p, t + 1, u + 2); set(r + R_ACT1_ALPHA, co, n);
            snprintf(n, sizeof(n), "%s.%d.block.%d.act1.beta", p, t + 1, u + 2); set(r + R_ACT1_BETA, co, n);
            snprintf(n, sizeof(n), "%s.%d.block.%d.conv1.conv.weight", p, t + 1, u + 2); set(r + R_CONV1_W, co * co * 7, n);
            snprintf(n, sizeof(n), "%s.%d.block.%d.conv1.conv.bias", p, t + 1, u + 2); set(r + R_CONV1_B, co, n);
            snprintf(n, sizeof(n), "%s.%d.block.%d.act2.alpha", p, t + 1, u + 2); set(r + R_ACT2_ALPHA, co, n);
            snprintf(n, sizeof(n), "%s.%d.block.%d.act2.beta", p, t + 1, u + 2); set(r + R_ACT2_BETA, co, n);
            snprintf(n, sizeof(n), "%s.%d.block.%d.conv2.conv.weight", p, t + 1, u + 2); set(r + R_CONV2_W, co * co, n);
            snprintf(n, sizeof(n), "%s.%d.block.%d.conv2.conv.bias", p, t + 1, u + 2); set(r + R_CONV2_B, co, n);
        }
    }
    set(T_DEC5_ALPHA, 96, "decoder.decoder.5.alpha");
    set(T_DEC5_BETA, 96, "decoder.decoder.5.beta");
    set(T_DEC6_W, 96ull * 7, "decoder.decoder.6.conv.weight");
    set(T_DEC6_B, 1, "decoder.decoder.6.conv.bias");
    g_table_ready = 1;
}

const char* orc_codec_tensor_name(int index) {
    build_table();
    return index >= 0 && index < ORC_CODEC_TENSORS ? g_names[index] : NULL;
}

uint64_t orc_codec_tensor_elements(int index) {
    build_table();
    return index >= 0 && index < ORC_CODEC_TENSORS ? g_elements[index] : 0;
}

/* ---- state ------------------------------------------------------------- */
static size_t residual_history(int stage, int unit) { return (size_t)kStageOut[stage] * 6 * kDilation[unit]; }

struct OrcCodecState {
    uint64_t position; /* neural frame position (CS:1260) */
    float frontend[2 * 512];
    float kv_k[LAYERS][HEADS][KV_WINDOW][HEAD_DIM];
    float kv_v[LAYERS][HEADS][KV_WINDOW][HEAD_DIM];
    float latent[2][6 * 1024];
    float dec_pre[6 * 1024];
    float* tail[4];        /* [stride][out] transposed-conv overlap (CS:1085-1113) */
    float* residual[4][3]; /* [6 d][channels] */
    float final_conv[6 * 96];
};

OrcCodecState* orc_codec_state_create(void) {
    OrcCodecState* s = (OrcCodecState*)calloc(1, sizeof(OrcCodecState));
    for (int t = 0; t < 4; ++t) {
        s->tail[t] = (float*)calloc((size_t)kStride[t] * kStageOut[t], sizeof(float));
        for (int u = 0; u < 3; ++u) s->residual[t][u] = (float*)calloc(residual_history(t, u), sizeof(float));
    }
    return s;
}

void orc_codec_state_reset(OrcCodecState* s) {
    s->position = 0;
    memset(s->frontend, 0, sizeof(s->frontend));
    memset(s->kv_k, 0, sizeof(s->kv_k));
    memset(s->kv_v, 0, sizeof(s->kv_v));
    memset(s->latent, 0, sizeof(s->latent));
    memset(s->dec_pre, 0, sizeof(s->dec_pre));
    memset(s->final_conv, 0, sizeof(s->final_conv));
    for (int t = 0; t < 4; ++t) {
        memset(s->tail[t], 0, (size_t)kStride[t] * kStageOut[t] * sizeof(float));
        for (int u = 0; u < 3; ++u) memset(s->residual[t][u], 0, residual_history(t, u) * sizeof(float));
    }
}

void orc_codec_state_destroy(OrcCodecState* s) {
    if (!s) return;
    for (int t = 0; t < 4; ++t) {
        free(s->tail[t]);
        for (int u = 0; u < 3; ++u) free(s->residual[t][u]);
    }
    free(s);
}

/* ---- GEMM (cuBLAS in the reference): y[m][n] = sum_k a[m][k] w[n][k] ---- */
typedef struct GemmJob {
    const float *a, *w, *bias;
    float* y;
    int m, n, k;
    int order;
} GemmJob;

static void gemm_range(void* p, int n0, int n1) {
    const GemmJob* g = (const GemmJob*)p;
    for (int i = 0; i < g->m; ++i) {
        const float* ai = g->a + (size_t)i * g->k;
        for (int j = n0; j < n1; ++j) {
            const float* wj = g->w + (size_t)j * g->k;
            float acc;
            if (g->order == 1) {
                double sum = 0.0;
                for (int t = 0; t < g->k; ++t) sum += (double)ai[t] * (double)wj[t];
                acc = (float)sum;
            } else {
                acc = 0.0f;
                for (int t = 0; t < g->k; ++t) acc = fmaf(ai[t], wj[t], acc);
            }
            if (g->bias) acc += g->bias[j]; /* add_bias_kernel, CS:407-412 */
            g->y[(size_t)i * g->n + j] = acc;
        }
    }
}

static void gemm(const float* a, const float* w, const float* bias, float* y, int m, int n, int k) {
    GemmJob g = {a, w, bias, y, m, n, k, orc_get_gemm_order()};
    orc_for_channels(n, (size_t)m * n * k, gemm_range, &g);
}

/* ---- frontend (CS:3321-3490) ------------------------------------------- */
static void frontend(const float* const* W, OrcCodecState* s, const uint16_t* codes, int frames, float* rvq,
                     float* preconv) {
    float semantic[MAX_FRAMES * 256], acoustic[MAX_FRAMES * 256], rest[MAX_FRAMES * 512];
    for (int f = 0; f < frames; ++f) {
        for (int cb = 0; cb < 16; ++cb) {
            const uint16_t code = codes[f * 16 + cb];
            const float* emb = cb == 0 ? W[T_RVQ_FIRST_EMB] : W[T_RVQ_REST_EMB + cb - 1];
            const float* usage = cb == 0 ? W[T_RVQ_FIRST_USAGE] : W[T_RVQ_REST_USAGE + cb - 1];
            const float u = fmaxf(usage[code], 1.0e-5f);
            for (int d = 0; d < 256; ++d) {
                const float v = emb[(size_t)code * 256 + d] / u; /* gather_codebook_kernel, CS:322-342 */
                if (cb == 0) semantic[f * 256 + d] = v;
                else if (cb == 1) acoustic[f * 256 + d] = v;
                else acoustic[f * 256 + d] = acoustic[f * 256 + d] + v;
            }
        }
    }
    gemm(semantic, W[T_RVQ_FIRST_PROJ], NULL, rvq, frames, 512, 256);
    gemm(acoustic, W[T_RVQ_REST_PROJ], NULL, rest, frames, 512, 256);
    for (int i = 0; i < frames * 512; ++i) rvq[i] += rest[i]; /* add_rvq_projection_kernel */
    /* causal_preconv_kernel, CS:356-384: k = 3 over two history frames */
    const float* w = W[T_PRECONV_W];
    for (int f = 0; f < frames; ++f) {
        for (int o = 0; o < 1024; ++o) {
            float value = W[T_PRECONV_B][o];
            for (int i = 0; i < 512; ++i) {
                for (int k = 0; k < 3; ++k) {
                    const int src = f - (2 - k);
                    const float x = src >= 0 ? rvq[src * 512 + i] : s->frontend[(2 + src) * 512 + i];
                    value = fmaf(w[((size_t)o * 512 + i) * 3 + k], x, value);
                }
            }
            preconv[f * 1024 + o] = value;
        }
    }
    /* update_frontend_history_kernel, CS:386-405 */
    for (int c = 0; c < 512; ++c) {
        if (frames == 1) {
            s->frontend[c] = s->frontend[512 + c];
            s->frontend[512 + c] = rvq[c];
        } else {
            s->frontend[c] = rvq[(frames - 2) * 512 + c];
            s->frontend[512 + c] = rvq[(frames - 1) * 512 + c];
        }
    }
}

/* ---- transformer (CS:2276-2540), one frame ------------------------------ */
static void rms_norm(const float* x, const float* w, float* out) {
    /* rms_norm_kernel, CS:414-434 (rsqrtf restated as 1/sqrtf) */
    float sq = 0.0f;
    for (int i = 0; i < HIDDEN; ++i) sq = fmaf(x[i], x[i], sq);
    const float scale = 1.0f / sqrtf(sq / (float)HIDDEN + 1.0e-5f);
    for (int i = 0; i < HIDDEN; ++i) out[i] = x[i] * scale * w[i];
}

static void transformer_frame(const float* const* W, OrcCodecState* s, const float* input, uint64_t position,
                              float* output) {
    float h[HIDDEN], h2[HIDDEN], n[HIDDEN], q[1024], k[1024], v[1024], attn[1024], proj[HIDDEN], gate[1024], up[1024];
    gemm(input, W[T_INPUT_PROJ_W], W[T_INPUT_PROJ_B], h, 1, HIDDEN, 1024);
    for (int l = 0; l < LAYERS; ++l) {
        const float* const* L = W + T_LAYER + 11 * l;
        rms_norm(h, L[L_IN_NORM], n);
        gemm(n, L[L_Q], NULL, q, 1, 1024, HIDDEN);
        gemm(n, L[L_K], NULL, k, 1, 1024, HIDDEN);
        gemm(n, L[L_V], NULL, v, 1, 1024, HIDDEN);
        /* apply_rope_kernel, CS:464-494: rotate-half pairs (d, d + 32) */
        for (int head = 0; head < HEADS; ++head) {
            for (int d = 0; d < 32; ++d) {
                const float frequency = 1.0f / powf(10000.0f, (float)(2 * d) / 64.0f);
                const float angle = (float)position * frequency;
                const float sine = sinf(angle), cosine = cosf(angle);
                const int a = head * 64 + d, b = a + 32;
                const float q1 = q[a], q2 = q[b], k1 = k[a], k2 = k[b];
                q[a] = q1 * cosine - q2 * sine;
                q[b] = q2 * cosine + q1 * sine;
                k[a] = k1 * cosine - k2 * sine;
                k[b] = k2 * cosine + k1 * sine;
            }
        }
        /* sliding_attention_kernel, CS:496-566 */
        const int slot = (int)(position % KV_WINDOW);
        for (int head = 0; head < HEADS; ++head) {
            memcpy(s->kv_k[l][head][slot], k + head * 64, 64 * sizeof(float));
            memcpy(s->kv_v[l][head][slot], v + head * 64, 64 * sizeof(float));
        }
        const uint64_t first = position + 1 > KV_WINDOW ? position + 1 - KV_WINDOW : 0;
        const int count = (int)(position - first + 1);
        for (int head = 0; head < HEADS; ++head) {
            float scores[KV_WINDOW];
            float maximum = -3.402823466e+38f;
            for (int i = 0; i < count; ++i) {
                const int src = (int)((first + (uint64_t)i) % KV_WINDOW);
                float score = 0.0f;
                for (int d = 0; d < 64; ++d) score = fmaf(q[head * 64 + d], s->kv_k[l][head][src][d], score);
                score *= 0.125f;
                scores[i] = score;
                maximum = fmaxf(maximum, score);
            }
            float denominator = 0.0f;
            for (int i = 0; i < count; ++i) {
                scores[i] = q3_expf(scores[i] - maximum);
                denominator += scores[i];
            }
            for (int d = 0; d < 64; ++d) {
                float result = 0.0f;
                for (int i = 0; i < count; ++i) {
                    const int src = (int)((first + (uint64_t)i) % KV_WINDOW);
                    result = fmaf(scores[i] / denominator, s->kv_v[l][head][src][d], result);
                }
                attn[head * 64 + d] = result;
            }
        }
        gemm(attn, L[L_O], NULL, proj, 1, HIDDEN, 1024);
        for (int i = 0; i < HIDDEN; ++i) h2[i] = h[i] + proj[i] * L[L_ATTN_SCALE][i]; /* CS:674-685 */
        rms_norm(h2, L[L_POST_NORM], n);
        gemm(n, L[L_GATE], NULL, gate, 1, 1024, HIDDEN);
        gemm(n, L[L_UP], NULL, up, 1, 1024, HIDDEN);
        for (int i = 0; i < 1024; ++i) v[i] = (gate[i] / (1.0f + q3_expf(-gate[i]))) * up[i]; /* CS:687-698 */
        gemm(v, L[L_DOWN], NULL, proj, 1, HIDDEN, 1024);
        for (int i = 0; i < HIDDEN; ++i) h[i] = h2[i] + proj[i] * L[L_MLP_SCALE][i];
    }
    rms_norm(h, W[T_NORM], n);
    gemm(n, W[T_OUTPUT_PROJ_W], W[T_OUTPUT_PROJ_B], output, 1, 1024, HIDDEN);
}

/* ---- latent upsampling (CS:1432-1667) ----------------------------------- */
static void convnext(const float* const* U, float* history, const float* input, int positions, float* output,
                     float* expanded) {
    /* depthwise_causal_kernel k = 7, CS:730-756 */
    for (int p = 0; p < positions; ++p) {
        for (int c = 0; c < 1024; ++c) {
            float r = U[U_DW_B][c];
            for (int k = 0; k < 7; ++k) {
                const int src = p - (6 - k);
                const float x = src >= 0 ? input[src * 1024 + c] : history[(6 + src) * 1024 + c];
                r = fmaf(U[U_DW_W][c * 7 + k], x, r);
            }
            output[p * 1024 + c] = r;
        }
    }
    /* update_causal_history_kernel, CS:758-776 */
    for (int hp = 0; hp < 6; ++hp) {
        const int combined = hp + positions;
        for (int c = 0; c < 1024; ++c) {
            history[hp * 1024 + c] = combined < 6 ? history[combined * 1024 + c] : input[(combined - 6) * 1024 + c];
        }
    }
    /* layer_norm_kernel eps 1e-6, CS:778-808 */
    for (int p = 0; p < positions; ++p) {
        float* row = output + p * 1024;
        float mean = 0.0f;
        for (int c = 0; c < 1024; ++c) mean += row[c];
        mean /= 1024.0f;
        float variance = 0.0f;
        for (int c = 0; c < 1024; ++c) {
            const float centered = row[c] - mean;
            variance = fmaf(centered, centered, variance);
        }
        const float scale = 1.0f / sqrtf(variance / 1024.0f + 1.0e-6f);
        for (int c = 0; c < 1024; ++c) row[c] = (row[c] - mean) * scale * U[U_NORM_W][c] + U[U_NORM_B][c];
    }
    gemm(output, U[U_PW1_W], U[U_PW1_B], expanded, positions, 4096, 1024);
    for (int i = 0; i < positions * 4096; ++i) {
        const float v = expanded[i];
        expanded[i] = 0.5f * v * (1.0f + erff(v * 0.7071067811865475f)); /* gelu_kernel, CS:860-866 */
    }
    gemm(expanded, U[U_PW2_W], U[U_PW2_B], output, positions, 1024, 4096);
    for (int p = 0; p < positions; ++p) {
        for (int c = 0; c < 1024; ++c) output[p * 1024 + c] = input[p * 1024 + c] + output[p * 1024 + c] * U[U_GAMMA][c];
    }
}

/* Transposed-convolution weights [in][out][taps] regrouped as [tap][in][out]
 * so that the loops below run along contiguous output channels; the fmaf
 * chain of each output element is unchanged (input channels in order). */
static float* taps_major(const float* w, int cin, int cout, int taps) {
    float* t = (float*)malloc((size_t)cin * cout * taps * sizeof(float));
    for (int i = 0; i < cin; ++i)
        for (int o = 0; o < cout; ++o)
            for (int k = 0; k < taps; ++k) t[((size_t)k * cin + i) * cout + o] = w[((size_t)i * cout + o) * taps + k];
    return t;
}

/* r[o] = fmaf(x[i], w[i][o], r[o]) over i in order, for every o */
static void chain_rows(const float* x, const float* w, int cin, int cout, float* r) {
    for (int i = 0; i < cin; ++i) {
        const float xi = x[i];
        const float* wi = w + (size_t)i * cout;
        for (int o = 0; o < cout; ++o) r[o] = fmaf(xi, wi[o], r[o]);
    }
}

typedef struct TransposeJob {
    const float *input, *taps, *bias, *tail;
    float* output;
    int cin, cout, stride, overlap;
} TransposeJob;

/* Output positions [op0, op1).  With overlap (kernel 2 * stride), position
 * ip * stride + phase takes tap stride + phase of input ip - 1 (or the stored
 * tail for ip == 0), then tap phase of input ip. */
static void transpose_range(void* p, int op0, int op1) {
    const TransposeJob* j = (const TransposeJob*)p;
    for (int op = op0; op < op1; ++op) {
        const int ip = op / j->stride, phase = op % j->stride;
        float* r = j->output + (size_t)op * j->cout;
        for (int o = 0; o < j->cout; ++o) r[o] = j->bias[o];
        if (j->overlap) {
            if (ip == 0) {
                for (int o = 0; o < j->cout; ++o) r[o] += j->tail[phase * j->cout + o];
            } else {
                chain_rows(j->input + (size_t)(ip - 1) * j->cin, j->taps + (size_t)(j->stride + phase) * j->cin * j->cout,
                           j->cin, j->cout, r);
            }
        }
        chain_rows(j->input + (size_t)ip * j->cin, j->taps + (size_t)phase * j->cin * j->cout, j->cin, j->cout, r);
    }
}

/* latent_transpose_kernel, CS:700-728: kernel 2, stride 2, no overlap */
static void latent_transpose(const float* const* U, const float* input, int positions, float* output) {
    float* taps = taps_major(U[U_CONV_W], 1024, 1024, 2);
    TransposeJob j = {input, taps, U[U_CONV_B], NULL, output, 1024, 1024, 2, 0};
    orc_for_channels(2 * positions, (size_t)2 * positions * 1024 * 1024, transpose_range, &j);
    free(taps);
}

/* ---- waveform decoder (CS:1669-2274) ------------------------------------ */
static void snake(const float* x, const float* alpha_p, const float* beta_p, int positions, int channels, float* out) {
    for (int p = 0; p < positions; ++p) {
        for (int c = 0; c < channels; ++c) {
            const float alpha = expf(alpha_p[c]), beta = expf(beta_p[c]); /* snake_beta_kernel, CS:882-898 */
            const float v = x[p * channels + c];
            const float sine = sinf(v * alpha);
            out[p * channels + c] = v + (sine * sine) / (beta + 1.0e-9f);
        }
    }
}

/* causal_im2col_kernel + update_causal_history_kernel + the GEMM (CS:1699-1782) */
static void causal_conv(const float* input, int positions, int cin, int cout, int kernel, int dilation, float* history,
                        const float* w, const float* bias, float* output) {
    const int hist = (kernel - 1) * dilation;
    const int width = cin * kernel;
    float* cols = (float*)malloc((size_t)positions * width * sizeof(float));
    for (int p = 0; p < positions; ++p) {
        for (int c = 0; c < cin; ++c) {
            for (int k = 0; k < kernel; ++k) {
                const int src = p - (kernel - 1 - k) * dilation;
                cols[(size_t)p * width + c * kernel + k] =
                    src >= 0 ? input[(size_t)src * cin + c] : history[(size_t)(hist + src) * cin + c];
            }
        }
    }
    if (hist > 0) {
        for (int hp = 0; hp < hist; ++hp) {
            const int combined = hp + positions;
            for (int c = 0; c < cin; ++c) {
                history[(size_t)hp * cin + c] =
                    combined < hist ? history[(size_t)combined * cin + c] : input[(size_t)(combined - hist) * cin + c];
            }
        }
    }
    gemm(cols, w, bias, output, positions, cout, width);
    free(cols);
}

/* transpose_overlap_neural_kernel + update_transpose_tail_neural_kernel,
 * CS:932-989, 1085-1113: kernel 2 * stride, stride, overlap tail */
static void decoder_transpose(const float* input, int positions, int cin, int cout, int stride, const float* w,
                              const float* bias, float* tail, float* output) {
    float* taps = taps_major(w, cin, cout, 2 * stride);
    TransposeJob j = {input, taps, bias, tail, output, cin, cout, stride, 1};
    orc_for_channels(positions * stride, (size_t)positions * stride * cout * cin * 2, transpose_range, &j);
    /* next tail: tap stride + phase of the last input, from zero */
    for (int phase = 0; phase < stride; ++phase) {
        float* r = tail + (size_t)phase * cout;
        for (int o = 0; o < cout; ++o) r[o] = 0.0f;
        chain_rows(input + (size_t)(positions - 1) * cin, taps + (size_t)(stride + phase) * cin * cout, cin, cout, r);
    }
    free(taps);
}

static void copy_trace(float* dst, const float* src, size_t count) {
    if (dst) memcpy(dst, src, count * sizeof(float));
}

int orc_codec_packet(const float* const* W, OrcCodecState* s, const uint16_t* codes, int frames, int16_t* pcm,
                     OrcCodecTrace* trace) {
    if (frames < 1 || frames > MAX_FRAMES) return -1;
    float rvq[MAX_FRAMES * 512], pre[MAX_FRAMES * 1024], tr[MAX_FRAMES * 1024];
    const int stop = trace ? trace->stop_after : 0;
    frontend(W, s, codes, frames, rvq, pre);
    if (trace) {
        copy_trace(trace->rvq, rvq, (size_t)frames * 512);
        copy_trace(trace->preconv, pre, (size_t)frames * 1024);
    }
    if (stop == 1) return 0;
    for (int f = 0; f < frames; ++f) transformer_frame(W, s, pre + f * 1024, s->position + (uint64_t)f, tr + f * 1024);
    s->position += (uint64_t)frames;
    if (trace) copy_trace(trace->transformer, tr, (size_t)frames * 1024);
    if (stop == 2) return 0;
    /* latent upsampling: 2 x (transposed conv x2, ConvNeXt) */
    const int latent = 4 * frames;
    float* la = (float*)malloc((size_t)latent * 1024 * sizeof(float));
    float* lb = (float*)malloc((size_t)latent * 1024 * sizeof(float));
    float* expanded = (float*)malloc((size_t)latent * 4096 * sizeof(float));
    const float* in = tr;
    int positions = frames;
    for (int st = 0; st < 2; ++st) {
        const float* const* U = W + T_UPSAMPLE + 11 * st;
        latent_transpose(U, in, positions, la);
        positions *= 2;
        convnext(U, s->latent[st], la, positions, lb, expanded);
        if (trace) copy_trace(st == 0 ? trace->latent1 : trace->latent2, lb, (size_t)positions * 1024);
        in = lb;
    }
    if (stop == 3) {
        free(la); free(lb); free(expanded);
        return 0;
    }
    /* waveform decoder */
    const size_t samples = (size_t)frames * 1920;
    float* cur = (float*)malloc(samples * 1536 * sizeof(float) / 4 + samples * 96 * sizeof(float));
    float* oth = (float*)malloc(samples * 1536 * sizeof(float) / 4 + samples * 96 * sizeof(float));
    float* tmp = (float*)malloc(samples * 96 * sizeof(float) + (size_t)latent * 1536 * sizeof(float));
    causal_conv(lb, positions, 1024, 1536, 7, 1, s->dec_pre, W[T_DEC0_W], W[T_DEC0_B], cur);
    int channels = 1536;
    float* const* checkpoint = trace ? trace->checkpoints : NULL;
    int result = 0;
    if (checkpoint) copy_trace(checkpoint[6], cur, (size_t)positions * channels);
    if (stop == 6) goto done;
    for (int t = 0; t < 4; ++t) {
        const float* const* S = W + T_STAGE + 28 * t;
        snake(cur, S[S_ALPHA], S[S_BETA], positions, channels, oth);
        decoder_transpose(oth, positions, channels, kStageOut[t], kStride[t], S[S_TCONV_W], S[S_TCONV_B], s->tail[t], cur);
        positions *= kStride[t];
        channels = kStageOut[t];
        for (int u = 0; u < 3; ++u) {
            const float* const* R = S + S_UNIT + 8 * u;
            snake(cur, R[R_ACT1_ALPHA], R[R_ACT1_BETA], positions, channels, oth);
            causal_conv(oth, positions, channels, channels, 7, kDilation[u], s->residual[t][u], R[R_CONV1_W], R[R_CONV1_B], tmp);
            snake(tmp, R[R_ACT2_ALPHA], R[R_ACT2_BETA], positions, channels, oth);
            causal_conv(oth, positions, channels, channels, 1, 1, NULL, R[R_CONV2_W], R[R_CONV2_B], tmp);
            for (size_t i = 0; i < (size_t)positions * channels; ++i) tmp[i] += cur[i]; /* add_residual_kernel */
            memcpy(cur, tmp, (size_t)positions * channels * sizeof(float));
        }
        if (checkpoint) copy_trace(checkpoint[7 + t], cur, (size_t)positions * channels);
        if (stop == 7 + t) goto done;
    }
    snake(cur, W[T_DEC5_ALPHA], W[T_DEC5_BETA], positions, 96, oth);
    if (checkpoint) copy_trace(checkpoint[11], oth, (size_t)positions * 96);
    if (stop == 11) goto done;
    causal_conv(oth, positions, 96, 1, 7, 1, s->final_conv, W[T_DEC6_W], W[T_DEC6_B], cur);
    if (checkpoint) copy_trace(checkpoint[12], cur, (size_t)positions);
    if (stop == 12) goto done;
    for (int i = 0; i < positions; ++i) cur[i] = fminf(1.0f, fmaxf(-1.0f, cur[i])); /* clamp_waveform_kernel */
    if (checkpoint) copy_trace(checkpoint[13], cur, (size_t)positions);
    if (stop == 13) goto done;
    for (int i = 0; i < positions; ++i) { /* waveform_to_pcm_kernel, CS:1133-1143 */
        const float scaled = roundf(cur[i] * 32767.0f);
        pcm[i] = (int16_t)fminf(32767.0f, fmaxf(-32768.0f, scaled));
    }
    result = positions;
done:
    free(la); free(lb); free(expanded); free(cur); free(oth); free(tmp);
    return result;
}
