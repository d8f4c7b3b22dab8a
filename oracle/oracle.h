// oracle.h - CPU restatement of sergqwer/geode's verify-step arithmetic.
//
// TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP implementation in geode_amd/: only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only to compare against or to time it
// as the CPU baseline. The product path (libgeode_verify.so) never links, loads or calls it.
//
// Every function restates a reference function; the citation is on each declaration (paths relative to the
// reference tree, engine/src/...). Pinning status per function: see the table at the top of oracle.cpp.
//
// Conventions: q4 matrices are in the reference pack's row layout (kernels.hpp:22-26, kernels.cpp:888-902): a row
// is cols/2 code bytes (value 2j in the low nibble of byte j, 2j+1 in the high one) followed by cols/16 E4M3
// scale bytes, one per 16-value block; value = kQ4[code] * E4M3(scale) * global. fp16 values travel as uint16 bits,
// bf16 values likewise.
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- portable seeded generator (not in the reference: the build's own, identical on every host) ----
uint64_t orc_hash(uint64_t seed, uint64_t i);
// out[i] = mean + sigma * N(0,1)_i, Box-Muller over orc_hash (double, rounded to float)
void orc_fill_normal(uint64_t seed, int64_t n, float mean, float sigma, float *out);
// out[i] uniform in (0, 1), 24-bit exact
void orc_fill_uniform(uint64_t seed, int64_t n, float *out);
uint16_t orc_f32_to_f16(float x);   // round to nearest even (static_cast<_Float16>)
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float x);  // round to nearest even

// ---- threads (the CPU baseline's row split: ThreadPool::parallel_for, chunks of 16 rows) ----
void orc_set_threads(int n);
int orc_threads(void);

// ---- q4 format ----
float orc_e4m3_value(uint8_t b);                         // kernels.cpp:39-52 (e4m3_table)
uint8_t orc_e4m3_byte(float x);                          // yue2_q4.cpp:72-83
void orc_q4_block(const float *x, float s2, uint8_t *scale_byte, uint8_t *codes16);   // yue2_q4.cpp:85-114
float orc_q4_global(const float *w, int64_t n);          // yue2_q4.cpp:338-343: max|w| * 1.25 / (15 * 448)
void orc_q4_pack(const float *w, int64_t rows, int64_t cols, float s2, uint8_t *out);   // yue2_q4.cpp:344-358
void orc_dequant_rows(const uint8_t *w, int64_t rows, int64_t cols, float global, float *out);   // kernels.cpp:1214

// ---- products ----
// exact: fp32 activations times the dequantized weights (kernels.cpp:1230-1250), rows [0, rows)
void orc_matvec_rows(const uint8_t *w, int64_t rows, int64_t cols, float global, const float *x, float *y);
// int8 activations per 16-value block (kernels.cpp:1254-1295)
void orc_quantize_activation(const float *x, int64_t cols, int8_t *q, float *scale, int32_t *bsum);
// int8 path (kernels.cpp:1304-1322)
void orc_matvec_rows_q(const uint8_t *w, int64_t rows, int64_t cols, float global, const int8_t *q,
                       const float *scale, float *y);
// bf16 rows times n fp32 tokens, eight partial sums in a fixed order (kernels.cpp:1446-1518)
void orc_matvec_bf16(const uint16_t *w, int64_t rows, int64_t cols, int n, const float *x, float *y);
void orc_rmsnorm(const float *x, const float *w, float *out, int n, float eps, int zero_centered);   // kernels.cpp:1520
// softmax, top-K by probability (ties to the lower index), weights renormalised in rank order (model.cpp:4021-4065)
void orc_route_topk(const float *logits, int E, int K, int *ids, float *weights);

// ---- layers (mode 0: the int8 path, the reference's default; mode 1: exact fp32 activations) ----
// C1: y[t] = down(silu(gate x[t]) * up x[t]) for M tokens (model.cpp:4126-4146, the dense MLP); x fp16 [M][H]
void orc_ffn_swiglu(const uint8_t *gate, const uint8_t *up, const uint8_t *down, float g_gate, float g_up,
                    float g_down, int H, int F, int M, const uint16_t *x_f16, int mode, float *y);

// One MoE layer (model.cpp:4123-4587): experts [E][block] in the pack's expert block layout (gate_up [2F x H] then
// down [H x F], pack.cpp:329-333), globals [E][2]; the shared expert as three matrices; router bf16 [E][H] or
// router_logits [M][E] given (C3); shared_gate bf16 [H]. out[M][H] the block's output (no residual); ids/wts
// [M][K]; gate[M] the shared gate after the sigmoid (may be NULL).
typedef struct {
    int H, E, K, F, SF;
    const uint8_t *experts;
    const float *expert_globals;
    const uint8_t *sh_gate, *sh_up, *sh_down;
    float sh_globals[3];
    const uint16_t *shared_gate;
    const uint16_t *router;
} orc_moe_weights;
void orc_moe_layer(const orc_moe_weights *w, int M, const float *h, const float *router_logits, int mode, float *out,
                   int *ids, float *wts, float *gate);

// ---- the full verify step (model.cpp:1483-1634, :3690-4019, :5235-5413) ----
typedef struct {
    int hidden, vocab, n_layers, n_experts, top_k, moe_ff, shared_ff;
    int n_heads, n_kv_heads, head_dim, rope_dim;
    float rope_theta, eps;
    int max_ctx;
    int attn_block;   // positions per attention block (model.hpp:458, kAttnBlock = 1024)
    int kv_int8;      // 1: the KV cache in int8, a scale a (position, KV head) (ModelOptions::kv_int8); 0: fp16
    // Gated DeltaNet layers (model.cpp:3497-3688; 0 heads: none): key / value heads and dims, the conv's width, and
    // per layer 1 for a GDN layer (else gated attention)
    int gdn_k_heads, gdn_v_heads, gdn_k_dim, gdn_v_dim, conv_kernel;
    unsigned char gdn_layers[256];
    // 1: an MTP layer (model.cpp:175-191): a full-attention layer at index n_layers (its KV after the main layers',
    // its experts at expert layer n_layers) behind fc, with its own final norm
    int mtp;
} orc_config;

// tensor kinds (shared numbering with include/geode_verify.h)
enum {
    ORC_EMBED = 0, ORC_LM_HEAD = 1, ORC_FINAL_NORM = 2, ORC_IN_NORM = 3, ORC_POST_NORM = 4, ORC_Q = 5, ORC_K = 6,
    ORC_V = 7, ORC_O = 8, ORC_Q_NORM = 9, ORC_K_NORM = 10, ORC_ROUTER = 11, ORC_SHARED_GATE = 12, ORC_EXPERT = 13,
    ORC_SH_GATE = 14, ORC_SH_UP = 15, ORC_SH_DOWN = 16, ORC_KV = 17,
    ORC_KV8 = 18,   // int8 KV: [K, V][max_ctx][nkv * hd] bytes
    ORC_KVS = 19,   // int8 KV: [K, V][max_ctx][nkv] float scales
    // a GDN layer's (model.cpp:129-138): in_proj_qkv q4 [2 kd + vd][H], in_proj_z q4 [vd][H], out_proj q4 [H][vd],
    // in_proj_a / in_proj_b bf16 [nv][H], A_log f32 [nv], dt_bias f32 [nv], conv1d f32 [2 kd + vd][K], norm f32 [dv]
    ORC_GDN_QKV = 20, ORC_GDN_Z = 21, ORC_GDN_OUT = 22, ORC_GDN_A = 23, ORC_GDN_B = 24, ORC_GDN_ALOG = 25,
    ORC_GDN_DTB = 26, ORC_GDN_CONV = 27, ORC_GDN_NORM = 28,
    ORC_GDN_CONV_ST = 29,   // the conv's state: [2 kd + vd][K - 1], the last K - 1 inputs oldest first
    ORC_GDN_S = 30,         // the recurrent state: [nv][dk][dv]
    // the MTP layer's own tensors (model.cpp:178-190; its decoder layer's: the kinds above at layer n_layers):
    // mtp.fc.weight q4 [H][2 H], mtp.norm / pre_fc_norm_embedding / pre_fc_norm_hidden f32 [H]
    ORC_MTP_FC = 31, ORC_MTP_NORM = 32, ORC_MTP_PRE_E = 33, ORC_MTP_PRE_H = 34
};

// fast_exp (kernels.hpp:142-163: Cephes' expf, the reduction by ln 2 in two parts and a degree-6 polynomial)
float orc_fast_exp(float x);
// One token of the gated delta rule on one value head (model.cpp:3499-3524): S [dk][dv] in place, S *= decay,
// delta = beta (v - S^T k), S += k delta^T, out = S^T q
void orc_gdn_step(float *S, int dk, int dv, const float *q, const float *k, const float *v, float decay, float beta,
                  float *out);

typedef struct orc_model orc_model;
// quant_kv_row (model.cpp:3766-3774): a KV head's row to int8, scale = amax / 127, q = clamp(nearbyint(x * (127 /
// amax)), -127, 127) (0 when amax = 0)
void orc_quant_kv_row(const float *x, int n, int8_t *q, float *scale);
orc_model *orc_model_create(const orc_config *cfg);
void orc_model_free(orc_model *m);
// A tensor's bytes (pack layout / f32 / bf16 / fp16 KV [2][max_ctx][nkv*hd]), their size and global scale(s)
// (expert: globals[0] gate_up, globals[1] down).
uint8_t *orc_model_tensor(orc_model *m, int kind, int layer, int expert, int64_t *bytes, float *globals);
// Seeded synthetic weights: N(0, sigma) quantized by the packer (router N(0, router_sigma) in bf16, norms N(0,
// 0.02), KV positions [0, ctx) N(0, 1) in fp16). fast != 0: random q4 bytes instead (codes uniform, scale bytes in
// [0x30, 0x48] as gpu_check.cpp:45-63, global 1/448) for timing only.
void orc_model_fill(orc_model *m, uint64_t seed, float sigma, float router_sigma, int ctx, int fast);
void orc_model_set_position(orc_model *m, int pos);
int orc_model_position(const orc_model *m);
// verify_n: n rows (tokens) at positions pos.. ; parents NULL = chain, else parents[0] = -1 and parents[i] < i (a
// draft tree in BFS order: row i sees the context, its ancestors and itself; its rotary position is pos + depth).
// logits [n][vocab]. The position advances by n. trace (may be NULL): per layer the routed ids [L][n][K].
int orc_model_verify(orc_model *m, const int32_t *tokens, int n, const int32_t *parents, int mode, float *logits,
                     int32_t *route_ids);
// orc_model_verify plus, per layer l, trace[l][4][n][hidden]: the residual stream into the layer, after the attention's
// residual add, the post-attention RMSNorm's output (the MoE block's input), and the MoE block's output (may be NULL)
int orc_model_verify_trace(orc_model *m, const int32_t *tokens, int n, const int32_t *parents, int mode,
                           float *logits, int32_t *route_ids, float *trace);
// verify_keep: kept rows stay (chain: rows 0..kept-1; tree: path[0..kept) of row indices, their KV moved to the
// kept slots); the position becomes the one before the verify plus kept.
int orc_model_keep(orc_model *m, int kept, const int32_t *path);
const orc_config *orc_model_config(const orc_model *m);
// The last verify's hidden rows after the final norm ([n][hidden], the MTP layer's input; n = the rows written)
int orc_model_hidden(const orc_model *m, float *out, int max_rows);
// Model::forward_mtp (model.cpp:4965-5039): n rows at MTP positions pos.., row t the pair (hidden row t, the token
// after it: toks[t]); hidden NULL = the last verify's final-normed rows (after a keep with a path: the path's rows).
// The layer's KV goes to slots pos..pos+n-1. logits (may be NULL: a prompt's pass, the KV only): the last row's,
// over the draft vocabulary when one is set, else the whole vocabulary.
int orc_model_mtp(orc_model *m, const int32_t *toks, int n, int pos, const float *hidden, int mode, float *logits);
// Model::draft (model.cpp:1295-1432): forward_mtp, draft = argmax of the last row's logits (the first maximum,
// mapped through the draft vocabulary), prob = its softmax probability summed in double (softmax_at, :1286-1292).
// logits may be NULL.
int orc_model_draft(orc_model *m, const int32_t *toks, int n, int pos, const float *hidden, int mode, float *logits,
                    int32_t *draft, float *prob);
// Model::draft_next (model.cpp:1434-1479): one more MTP row at position pos from the last MTP pass's normed output
// (its last row) and the token tok (the draft it made)
int orc_model_draft_next(orc_model *m, int32_t tok, int pos, int mode, float *logits, int32_t *draft, float *prob);
// The draft head (model.cpp:803-827): lm_head's rows of ids[0..n) (draft_vocab.bin); n = 0: the whole vocabulary
int orc_model_set_draft_vocab(orc_model *m, const int32_t *ids, int n);
// seconds of the last verify spent in the layers and in the final norm + lm_head
void orc_model_last_times(const orc_model *m, double *t_layers, double *t_head);

// ---- a conversation's state in the reference's file format (state.cpp, Model::save_state / load_state) ----
typedef struct {
    uint64_t pack_print;       // the pack's print folded into the fingerprint (0: taken as 1)
    uint64_t conv_id;
    int32_t extra, rope_delta;
    int32_t has_mtp, has_vision;   // the fingerprint's flags
    float *hidden;             // [hidden] or NULL: the last hidden state (written when has_mtp and the position > 0)
    int32_t has_hidden;        // load: the file held one and `hidden` received it
} orc_state_info;
uint64_t orc_fnv1a(const void *data, size_t n, uint64_t seed);   // state.cpp:71-75 (seed 1469598103934665603)
// Model::save_state (state.cpp:251-371) of the oracle model's position and KV cache; 0 or -1 with err
int orc_state_save(orc_model *m, const char *path, int append, const orc_state_info *info, char *err, int err_len);
// Model::load_state (state.cpp:373-463): the position becomes the saved one (0 on failure)
int orc_state_load(orc_model *m, const char *path, orc_state_info *info, char *err, int err_len);

// ---- sampling and acceptance ----
// Sampler::sample (sampler.cpp:16-50) with the uniform injected: u in [0, 1) stands for
// uniform_real_distribution<double>(0, kept) = kept * u. cap: candidates when top_k is off (1024 in the reference;
// 0 = the full vocabulary).
int orc_sample(const float *logits, int n, float temperature, float top_p, int top_k, int cap, double u);
// The reference's own stream: mt19937_64 seeded once, `draws` samples of the same row (for the _ref comparison)
void orc_sample_seeded(const float *logits, int n, float temperature, float top_p, int top_k, uint64_t seed,
                       int draws, int32_t *out);
// Sample-and-match over a verified chain (geode.cpp:318-374): batch = [tok, d1..d_{n-1}]; each row sampled with
// its uniform u[i]; a draft stands while row i samples exactly it. out: the tokens emitted (stood drafts, then the
// first sampled token that is no draft). Returns how many; *kept = the rows that stay (verify_keep's argument).
// The same with the generate loop's presence penalty and stop tokens (geode.cpp:236-255, :331-350): seen (the answer's
// tokens so far) lose presence_penalty in each row's logits (modified in place) before it is sampled, every sampled
// token joining seen; a draft stands only if it is no stop token either.
int orc_accept_match_ex(float *logits, int V, const int32_t *batch, int n, float temperature, float top_p, int top_k,
                        int cap, const double *u, const int32_t *seen, int n_seen, float presence_penalty,
                        const int32_t *stop, int n_stop, int32_t *out, int *kept);
int orc_accept_match(const float *logits, int V, const int32_t *batch, int n, float temperature, float top_p,
                     int top_k, int cap, const double *u, int32_t *out, int *kept);
// The textbook rule (Leviathan et al. 2023, Alg. 1). Not in the reference (which is sample-and-match above).
// p_i = nucleus(softmax(target_i / T), top_p), q_i likewise from draft_i. Draft i: d_i = argmax q_i (greedy) or
// sampled from q_i with u_draft[i]; accepted iff u_acc[i] * q_i(d_i) < p_i(d_i) (greedy: argmax p_i == d_i). At the
// first rejection the token comes from max(0, p_i - q_i) (inverse CDF in index order, uniform u_res); when all k
// stand, a bonus token from p_k (u_res). out: accepted drafts then the extra token; returns their count.
int orc_accept_textbook(const float *target, const float *draft, int V, int k, float temperature, float top_p,
                        int greedy, const float *u_draft, const float *u_acc, float u_res, int32_t *out);
// The nucleus used above, for tests: probabilities over the whole vocabulary (0 outside the nucleus)
void orc_nucleus_probs(const float *logits, int V, float temperature, float top_p, double *probs);

#ifdef __cplusplus
}
#endif
