// step.hpp - the verify step as one persistent kernel (step.hip): what it reads from the model, and the host entry.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "model.hpp"

namespace gv {

// One layer's weights as the persistent kernel reads them (device copies of LayerW's pointers and globals)
struct LayerDev {
    const uint8_t *qkv_c, *qkv_s, *o_c, *o_s;
    float g_q, g_k, g_v, g_o;
    const float *in_norm, *post_norm, *q_norm, *k_norm;
    const uint16_t *router;
    const uint8_t *gu_c, *gu_s, *dn_c, *dn_s;
    const float *eglob;
    _Float16 *kv;
};

// The skinny products' split: a product of K values is ranges of NS super-chunks (128 values) each, one wave a
// range, their sums added in range order; a pass is R ranges whose sum is applied before the next pass's (the
// per-launch K limit of the per-phase kernels, gemv_q4 in q4.hip), so both paths add in the same order.
struct ProdShape {
    int NS, R, P;
};

struct StepDev {
    const LayerDev *layers;
    int n_layers, H, V, E, K, F, nh, nkv, hd, half, max_rows;
    float eps;
    int64_t slots;   // KV positions a layer holds
    int nb_max;      // attention blocks: the stride of the partials
    int qkv_rows;
    size_t gu_cs, gu_ss, dn_cs, dn_ss;
    const uint8_t *emb_c, *emb_s;
    float emb_g;
    const uint8_t *lm_c, *lm_s;
    float lm_g;
    const float *final_norm, *rope_cos, *rope_sin;
    const StepParams *sp;
    // exchanged between workgroups, by device-coherent loads and stores: one arena (one buffer descriptor), byte
    // offsets of its parts
    uint8_t *arena;
    uint32_t arena_bytes; // the descriptor's range: offsets at or past it read 0 and write nothing
    uint32_t o_x;         // [M][H] fp32: the residual stream
    uint32_t o_qkv;       // [M][qkv_rows] fp32
    uint32_t o_rlog;      // [M][E + 1] fp32: router logits (the shared expert's gate last)
    uint32_t o_parts;     // [M][nh][nb_max][hd + 2] fp32: attention partials
    uint32_t o_y;         // [picks][H] fp32: the experts' outputs
    uint32_t o_logits;    // [M][V] fp32
    uint32_t o_act_h;     // [M] the products' operands of the normalized rows (input, post-attention or final norm)
    uint32_t o_act_core;  // [M] the output projection's operands
    uint32_t o_act_m;     // [picks] the down products' operands (SwiGLU rows)
    int32_t *route_ids;   // [n_layers][max_rows][K]
    RouteState *route;    // [n_layers]: workgroup 0's route, for the per-phase kernels' replays
    unsigned *flags, *rel, *err;
    uint64_t *stamps;    // null, or [grid][step_barriers][2]: each workgroup's clock (s_memrealtime, 100 MHz) when it
                         // arrives at a barrier and when it leaves the wait (a measurement aid)
    ProdShape sh_h, sh_o, sh_f;   // K = H (qkv, experts' gate|up, lm_head), K = nh hd (o), K = F (down)
};

// barriers one step takes: one after the embedding, eight a layer
inline unsigned step_barriers(int n_layers) { return 1u + 8u * static_cast<unsigned>(n_layers); }

struct Model;
// whether the persistent kernel takes this model at M rows (its product shapes and LDS fit); why not in `why`
bool step_supported(const Model &m, int M, const char **why);
int step_setup(Model &m);                              // device copies of the layer pointers, exchange buffers
int step_run(Model &m, int M, hipStream_t st);         // the whole verify step as one launch
int step_check(Model &m);                              // nonzero (and the error set) if a launch reported a timeout
int step_invalidate(Model &m);                         // after an adoption: the step's arguments are rebuilt
int step_trace(Model &m, bool on);                     // the barrier clock stamps on (allocated) or off
int64_t step_trace_read(Model &m, uint64_t *out, int64_t n);   // the last step's stamps; the count copied

}  // namespace gv
