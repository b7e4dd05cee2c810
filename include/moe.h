/* moe.h: the C ABI of the mixture-of-experts ops on MI355X (gfx950), in libdense_reader.so beside dense_reader.h.
 *
 * A MoE layer reads only the experts each token routed to. The expert ids stay on the device: every launch reads
 * them there, so nothing goes to the host and a HIP graph can capture the whole layer. The experts' weights are
 * dense_reader bfloat4_b weights (dr_pack), one after another in memory:
 *   gate/up: expert e's gate weight [K = H, N = I] at codes + e * codes_stride, its up weight at codes_up + e *
 *            codes_stride (exponents likewise, exps_stride);
 *   down:    expert e's weight [K = I, N = H] at codes + e * codes_stride.
 *
 * Reference interfaces replaced (XylolabsInc/tensix-kernels, paths relative to its root):
 *   dr_moe_matmul, mode DR_MOE_GATE_UP       <- moe/moe8.py:710-817 gate_up and its kernels moe_gu_reader.cpp,
 *                                               moe_gu2_reader.cpp, moe_gu_compute.cpp, moe_gu_writer.cpp
 *   dr_moe_matmul, mode DR_MOE_DOWN          <- moe/moe8.py:820-910 down and moe_dn_*.cpp, moe_dn2_*.cpp
 *   dr_moe_matmul, mode DR_MOE_GATE_UP_ROWS  <- moe/moe8.py:928-1037 gate_up_rows and moe_gur_*.cpp, moe8_rows.h
 *   dr_moe_matmul, mode DR_MOE_DOWN_ROWS     <- moe/moe8.py:1040-1136 down_rows and moe_dnr_*.cpp
 *   dr_moe_workspace_bytes                   <- (no counterpart: split K meets in caller memory, as dr_workspace_bytes)
 *   dr_moe_route                             <- moe/moe8.py:1139-1253 route and moe_route.cpp
 */
#ifndef DR_MOE_H
#define DR_MOE_H

#include <stdint.h>

#include "dense_reader.h"

#ifdef __cplusplus
extern "C" {
#endif

/* the expert gather of a launch */
#define DR_MOE_GATE_UP 1      /* one row: output slot s (columns s * I ..) from expert ids[0][s] */
#define DR_MOE_DOWN 2         /* one row: x's slot s (columns s * I ..) times expert ids[0][s]'s rows, summed */
#define DR_MOE_GATE_UP_ROWS 3 /* up to 32 rows: output block q (columns q * I ..) from the q-th expert of the union */
#define DR_MOE_DOWN_ROWS 4    /* up to 32 rows: x's block q times the q-th expert of the union's rows, summed */

/* GLU activations (dr_launch.act) */
#define DR_ACT_SILU 0
#define DR_ACT_GELU_TANH 1
#define DR_ACT_SWIGLU_OAI 2 /* min(g, 7) * sigmoid(1.702 min(g, 7)) * (clamp(u, -7, 7) + 1) */

typedef struct dr_moe {
    int32_t mode;          /* DR_MOE_* */
    const void* ids;       /* [id_rows][ld_ids] expert ids, uint16 (ids32 0) or uint32 */
    int32_t ids32;
    int32_t ld_ids;
    int32_t slots;         /* k, ids a row: 1 .. 16 */
    int32_t id_rows;       /* rows of ids: 1 for the one-row modes, R (1 .. 32) for the rows modes */
    int32_t experts;       /* E (the rows modes: 1 .. 1024); an id >= E chooses no expert */
    const void* w;         /* routing weights [id_rows][ld_w] bf16 (gate/up modes) */
    int32_t ld_w;
    int32_t expert_n;      /* gate/up modes: I, an expert's output columns */
    int32_t expert_k;      /* down modes: I, an expert's rows (x's block width) */
    int64_t codes_stride;  /* bytes from one expert's codes to the next */
    int64_t exps_stride;   /* bytes from one expert's exponents to the next */
    const void* bias;      /* gate/up modes: [E][2][expert_n] bf16, the gate's then the up's, or NULL */
} dr_moe;

/* The expert-gathered matmul. The launch describes one expert's weight (segment 0, bfloat4_b, expert 0's pointers)
 * and the rest as for dr_matmul:
 *   DR_MOE_GATE_UP (rows 1) and DR_MOE_GATE_UP_ROWS: segment glu 2 (codes = gate, codes_up = up), n = I, k = H; y
 *     [m][ldy] bf16 gets act(x G_e + b_g) * (x U_e + b_u) times the row's routing weight for e at columns s * I ..
 *     (slot s) or q * I .. (union index q, 0 where the row did not choose e). Slots whose id is >= E are written as
 *     zeros; union blocks past the union are not written.
 *   DR_MOE_DOWN (rows 1) and DR_MOE_DOWN_ROWS: segment glu 0, n = H; x [m][ldx] holds slot s's (union index q's) I
 *     values at s * I (q * I); k = its columns (slots * I, or the union's bound min(E, R * slots) * I); y [m][ldy]
 *     bf16 or fp32 = the sum over the slots (union) of the block times the expert's weight. Slots whose id is >= E
 *     and blocks past the union add nothing.
 * The union is the distinct ids < E of ids' first id_rows rows, in increasing order, computed by every workgroup.
 * dr_launch.act: DR_ACT_*; no residual, top-k or scales. Allocates nothing. */
int64_t dr_moe_workspace_bytes(const dr_launch* launch, const dr_moe* moe);
int dr_moe_matmul(const dr_launch* launch, const dr_moe* moe);

/* The router's top k of logits [rows][ld_logits] fp32 (columns 0 .. experts - 1; rows <= 32, experts <= 1024 and a
 * multiple of 32), written whole into ids [rows][ld_ids] (uint16 or uint32) and w [rows][ld_w] bf16, slots in
 * decreasing order of the pick's key, the lower id first among equal keys:
 *   kind 0 (softmax): keys the logits; w the softmax over the k picked logits;
 *   kind 1 (sigmoid): keys sigmoid(logit) + bias[e] (bias fp32 [experts], or NULL: keys the logits); w the picks'
 *     sigmoids over their sum (norm 0: not divided).
 * n_group > 0 (sigmoid with a bias): experts in n_group groups in order, a group's score the sum of its two largest
 * keys, the topk_group best groups kept (the lower group first among equal scores), the top k of their experts.
 * Every weight times scale; rounded to bf16 at the end. slot >= 0: slot k of every row gets that id at weight 1.0.
 * shared (bf16 [rows][ld_shared] or NULL): sigmoid(logits[r][experts]). Keys and weights in double. */
typedef struct dr_route {
    const float* logits;
    int32_t rows, ld_logits, experts, k;
    int32_t kind;          /* 0 softmax, 1 sigmoid */
    const float* bias;     /* [experts] or NULL */
    void* ids;
    int32_t ids32, ld_ids;
    void* w;               /* bf16 */
    int32_t ld_w;
    void* shared;          /* bf16 or NULL */
    int32_t ld_shared;
    double scale;
    int32_t norm;
    int32_t n_group, topk_group;
    int64_t slot;          /* -1: none */
    void* stream;
} dr_route;

int dr_moe_route(const dr_route* route);

/* dr_moe_route of one token (route->rows 1) and dr_moe_matmul's DR_MOE_GATE_UP over its picks, in one launch: every
 * workgroup routes the token itself (the router's code: the same ids and weights bit for bit) and gathers its slot's
 * expert; workgroup 0 writes ids and w as dr_moe_route does, for the down launch and the caller. route's ids, w,
 * ids32 and experts are moe's; moe->slots is route->k (+ 1 with a slot); experts at most 256 (DR_ERANGE beyond: route
 * with dr_moe_route, then dr_moe_matmul). The workspace is dr_moe_workspace_bytes(
 * launch, moe)'s. Replaces the pair route (moe/moe8.py:1139-1253) then gate_up (moe/moe8.py:710-817): no kernel
 * boundary between them. */
int dr_moe_route_gate_up(const dr_launch* launch, const dr_moe* moe, const dr_route* route);

#ifdef __cplusplus
}
#endif

#endif
