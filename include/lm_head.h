/* lm_head.h: the C ABI of the LM head's pick on MI355X (gfx950), in libdense_reader.so beside dense_reader.h.
 *
 * An LM head run as dense_reader matmuls with top-k records (dr_matmul's dr_topk, bf16 keys) leaves, per row, the
 * best candidates of every 32-column tile of the vocabulary. These entry points turn the records into token ids on the
 * device, with nothing read back: per row an output page of 32 uint32 words, [token, the device's own best id, the
 * valid candidates' count, 0 ...].
 *
 * Reference interfaces replaced (XylolabsInc/tensix-kernels, paths relative to its root):
 *   dr_head_pick         <- lm_head_topk/head_pick.py:101-220 pick() and its kernels head_pick_reader.cpp,
 *                           head_pick_compute.cpp, head_pick_writer.cpp (the best `top` candidates by key, their exact
 *                           logits from the bf16 head rows, the pick of lmhead.py:40-46 pick_token)
 *   dr_head_pick_records <- lm_head_topk/head_pick.py:241-329 pick_records() and head_pick_records.cpp (the best
 *                           record by the device's own logit, through a token map)
 *
 * Both take plain device pointers and a hipStream_t (as void*), allocate nothing, and return DR_OK or a DR_E* status
 * of dense_reader.h. Many records are selected by several workgroups a row that meet in a workspace of
 * dr_topk_merge_workspace_bytes(n_records, rows, k) bytes (dense_reader.h; zeroed once by the caller, its counters
 * left at zero by every launch; launches sharing one must not overlap in time).
 */
#ifndef LM_HEAD_H
#define LM_HEAD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* records [n_records][2 * rows * k] uint32 (dr_topk's bf16 records: keys, then ids); row r of x [rows][ldx] bf16
 * and the head table head [>= vocab][ld_head] bf16 (one row a token, dim columns used). Per row r < rows: the best
 * `top` (1 .. 32) valid slots by key, the earlier slot (record by record, slot by slot) first among equal keys; a slot
 * is valid when its key is not 0 and its id is below vocab. Their logits x[r] . head[id] summed in float32 (rounded to
 * bf16 with round_bf16), and the token is the lowest id among the largest logits, a NaN counting as the largest.
 * out [32][32] uint32: row r = [token (0 when no slot is valid), the first candidate's id (0xFFFFFFFF when none), the
 * candidates' count, 0 ...]. ids_out (or NULL): row 0's token also into ids_out[0]. rows <= 32; dim a multiple of 8;
 * x, head 16-byte aligned with ldx, ld_head multiples of 8. */
int dr_head_pick(const void* records, int n_records, int rows, int k, int top, int round_bf16, const void* x, int ldx,
                 int dim, const void* head, int64_t ld_head, int64_t vocab, void* out, void* ids_out, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* The records' pick with no rescore: per row r < rows, the valid slot of the largest key (a NaN's key above all, -0's
 * equal to +0's), the earliest among equals; its id mapped through token_map (int32 [>= vocab], or NULL: the id).
 * out [32][32] uint32: row r = [token, the id, the valid slots' count, 0 ...] ([0, 0xFFFFFFFF, 0] when none).
 * ids_out (or NULL): row 0's token also into ids_out[0]. */
int dr_head_pick_records(const void* records, int n_records, int rows, int k, int64_t vocab, const void* token_map,
                         void* out, void* ids_out, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif
