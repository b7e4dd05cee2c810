/* dense_reader.h: the C ABI of the MI355X (gfx950) dense_reader decode matmul.
 *
 * A weight-streaming matmul y = x @ w (* scale) for decode: x bf16 [M, K], w a block-float (bfloat8_b, bfloat4_b)
 * or bf16 weight [K, N] packed once into this library's HBM layout, fp32 accumulation, output bf16 or fp32, with the
 * fused output stages of the reference (per-column scales, SwiGLU/GeGLU, residual add, fp32 output, top-k records)
 * and block lists (up to four weights written into one output by one launch).
 *
 * Every entry point takes plain device pointers and sizes and a hipStream_t (as void*), allocates nothing, and
 * returns 0 or a DR_E* status (dr_status_string names it). Work is enqueued on the stream; nothing synchronises.
 *
 * Reference interfaces replaced (XylolabsInc/tensix-kernels, paths relative to its root):
 *   dr_pack        <- dense_reader/linear.py:144-156 native_weight's conversion (ttnn.from_torch(..., dtype,
 *                     TILE_LAYOUT)) and its column scale division (linear.py:149-151)
 *   dr_unpack      <- dense_reader/linear.py:159-163 block_float / ttnn.to_torch of a weight (the held values)
 *   dr_matmul      <- dense_reader/linear.py:828-1070 _launch's ttnn.generic_op(ios, ProgramDescriptor) with the
 *                     kernels dense_reader.cpp, dense_compute.cpp and dense_writer.cpp
 *   dr_topk_merge  <- the host merge of top-k records, dense_reader/linear.py:747-768 (records_host) followed by a
 *                     best-k selection as lm_head_topk/lmhead.py:212-239 does on the host
 *   dr_topk_merge_workspace_bytes <- (no counterpart: the merge runs on the host there)
 *   dr_plan        <- dense_reader/linear.py:455-495 choose/plan (the work split, for inspection only)
 *   dr_pack_int4, dr_int4_scales_bytes, dr_pack_int4_scales <- int4/w4a16.py:69-97 int4_weight / group_scales
 *                     (the int4 weight's conversions; dr_matmul with a DR_INT4 segment replaces w4a16_linear)
 *   dr_workspace_bytes <- (no counterpart: the reference's per-core accumulators live in L1 circular buffers,
 *                     linear.py:937; here a K split over workgroups meets in caller-provided device memory)
 */
#ifndef DENSE_READER_H
#define DENSE_READER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* weight formats (the reference's ttnn.bfloat8_b, ttnn.bfloat4_b, ttnn.bfloat16; DR_INT4 the W4A16 weight of
 * int4/w4a16.py: codes q in -7..7 with one bf16 scale per output column and 32 inputs, the weight q * s) */
#define DR_BFP8 0
#define DR_BFP4 1
#define DR_BF16 2
#define DR_INT4 3
/* bfloat4_b with its shared exponents along K (each tile's blocks transposed: an exponent for 16 consecutive K at one
 * N), the layout of moe8.pack(kblock=True) (moe/moe8.py:117-172, 507-527): dr_pack, dr_unpack and the expert gather of
 * dr_moe_matmul (include/moe.h) take it; dr_matmul does not. */
#define DR_BFP4_KB 4

/* statuses */
#define DR_OK 0
#define DR_EINVAL 1   /* an argument outside what the op takes (Python: AssertionError / ValueError) */
#define DR_EHIP 2     /* a HIP runtime error (Python: RuntimeError) */
#define DR_ERANGE 3   /* a size beyond a documented limit */

/* Geometry of a packed weight of K rows (in) and N columns (out):
 *   k_pad = K rounded up to 256, n_pad = N rounded up to 32 (or a multiple the caller asks for);
 *   codes: n_pad / 16 panels x k_pad values; bytes = k_pad * n_pad (bfp8), k_pad * n_pad / 2 (bfp4),
 *          2 * k_pad * n_pad (bf16);
 *   exps:  one byte per (panel, k): k_pad * n_pad / 16 bytes (bfp8, bfp4; none for bf16), each panel's in groups
 *          of 256 k ordered as the kernels read them (dense_reader.hip describes the layout). */
int64_t dr_codes_bytes(int fmt, int k_pad, int n_pad);
int64_t dr_exps_bytes(int fmt, int k_pad, int n_pad);

/* Pack w [N=out rows][K=in columns] fp32 (device, row stride ld_w elements) as the weight [K, N] in format fmt:
 * each 16 output columns at one k share one exponent (the reference's face row), values rounded as the reference's
 * host conversion does. col_div (device [N] fp32, or NULL): row n of w divided by col_div[n] first (native_weight's
 * col_scale). Columns n >= N and rows k >= K up to n_pad, k_pad hold zeros. */
int dr_pack(const float* w, int64_t ld_w, int n, int k, int fmt, const float* col_div, void* codes, void* exps,
            int n_pad, int k_pad, void* stream);

/* Pack int4 codes q [N][ld_q] int8 (-7..7; device) as a DR_INT4 weight [K, N]: bfloat4_b's code layout (nibbles
 * u = q + 8), no exponents; zeros past N and K up to n_pad, k_pad (replaces int4/w4a16.py:69-86 int4_weight's
 * conversion). */
int dr_pack_int4(const int8_t* q, int64_t ld_q, int n, int k, void* codes, int n_pad, int k_pad, void* stream);

/* Lay out the group scales s [N][ld_s] bf16 (one per output column and 32 inputs; device) for a DR_INT4 weight:
 * out [n_pad / 16][k_pad / 128][4][16] bf16, zeros past N and K (dr_int4_scales_bytes; replaces int4/w4a16.py:89-97
 * group_scales). */
int64_t dr_int4_scales_bytes(int k_pad, int n_pad);
int dr_pack_int4_scales(const uint16_t* s, int64_t ld_s, int n, int k, void* out, int n_pad, int k_pad, void* stream);

/* The held values of a packed weight: out [K][ld_out] fp32 (device), columns 0 .. n-1. */
int dr_unpack(const void* codes, const void* exps, int fmt, int n, int k, int n_pad, int k_pad, float* out,
              int64_t ld_out, void* stream);

/* One weight (or gate/up pair) of a launch: its output columns [col0, col0 + n_out) of y, n_out = n, or n / 2
 * for an interleaved GLU weight (glu 1). */
typedef struct dr_segment {
    int32_t fmt;        /* DR_BFP8, DR_BFP4, DR_BF16 */
    int32_t n;          /* the weight's columns (glu 1: 2 * the output's, gate and up tiles alternating) */
    int32_t n_pad;      /* the packed weight's padded columns (a multiple of 32) */
    int32_t glu;        /* 0 none; 1 interleave_glu weight; 2 gate in codes/exps, up in codes_up/exps_up */
    const void* codes;
    const void* exps;
    const void* codes_up;
    const void* exps_up;
    const void* scale;    /* per weight column scales [n] or NULL (unit); DR_INT4: its group scales
                             (dr_pack_int4_scales), required */
    const void* scale_up; /* glu 2: the up weight's scales or NULL */
    int32_t scale_f32;    /* scales are fp32 (1) or bf16 (0) */
    int32_t col0;         /* first output column in y, a multiple of 32 */
} dr_segment;

/* Top-k records: the launch's 32-column output tiles in groups of G consecutive tiles, one record for each group at
 * index slot0 + group, holding, for each of the first `rows` rows, the best k values of the group's columns (highest
 * first, ties to the lower column), written as rows * k keys then rows * k ids (uint32 words). G = 1 (a record a
 * tile) unless the launch has more tiles than max_records; then G = ceil(tiles / max_records), so that a launch
 * writes at most max_records records, as the reference's writes at most one a core of its grid (a caller that sizes
 * each block's records by the grid's cores, lm_head_topk/lmhead.py:102-103, stays within them). fp32 0: keys are the
 * reference's bf16 keys of the bf16 output (0 empty) and ids base + column (0xFFFFFFFF empty); fp32 1: keys are the
 * fp32 scores' bits (-inf empty) and ids int32 (-1 empty). Grouped launches (G > 1) stage every tile's record in the
 * workspace (dr_workspace_bytes), rank the groups in a second kernel on the stream, and take at most 1024 = G * k
 * candidates a row. */
typedef struct dr_topk {
    void* records;       /* [records_cap][2 * rows * k] uint32, or NULL: no top-k */
    int32_t k;           /* 1 .. 32 */
    int32_t rows;        /* 1 .. 32, at most the launch's rows */
    int32_t slot0;
    int32_t records_cap;
    int32_t n_valid;     /* output columns taking part (columns >= n_valid never enter) */
    int64_t base;        /* id of output column 0 */
    int32_t write_y;     /* 0: y is not written */
    int32_t fp32;
    int32_t max_records; /* records the launch writes at most (the caller's records per block); 0: one a tile */
} dr_topk;

typedef struct dr_launch {
    const void* x;       /* [m][ldx] bf16, 16-byte aligned, ldx a multiple of 8 (rows are read 16 bytes at a time) */
    int32_t m, k, ldx;
    void* y;             /* [m][ldy] bf16 or fp32 */
    int32_t ldy;
    int32_t y_f32;
    const void* residual; /* [m][ldr] bf16 or NULL */
    int32_t ldr;
    int32_t residual_mode; /* 1 epilogue: y = acc + r; 2 preload: the sum starts at r */
    int32_t act;         /* GLU activation: 0 silu (SwiGLU), 1 gelu_tanh (GeGLU) */
    int32_t nseg;        /* 1 .. 4 */
    dr_segment seg[4];
    dr_topk topk;
    void* workspace;     /* device memory for split K (dr_workspace_bytes), zeroed once by the caller; or NULL */
    int64_t workspace_bytes;
    void* stream;        /* hipStream_t */
} dr_launch;

/* dr_matmul_noalloc's own device workspace: DR_SCRATCH_BYTES a GPU, from the first call on a device until the process
 * ends. */
#define DR_SCRATCH_BYTES (8 << 20)

/* Bytes of workspace the launch needs (0: none; a K long enough to split over several workgroups a tile needs some;
 * -1: the launch is invalid). The workspace is zeroed once when allocated; every launch leaves its counters at zero,
 * and they lie at the same place whatever the launch's shape, so launches of any shape (dr_matmul's and
 * dr_moe_matmul's) can share one, but not with the top-k merge or the head pick. Launches that share one workspace
 * must not overlap in time (one stream). */
int64_t dr_workspace_bytes(const dr_launch* launch);

/* y = the launch's fused matmul. Allocates nothing. A DR_INT4 weight goes alone (one segment, no GLU, residual or
 * top-k) and takes its rows two at a time (int4/w4a16.py:170-253 w4a16_linear takes one token). */
int dr_matmul(const dr_launch* launch);

/* dr_matmul without a caller workspace: a launch that needs one (dr_workspace_bytes > 0) uses the library's own,
 * a static device array of DR_SCRATCH_BYTES on each GPU (dr_scratch_bytes), so the call allocates nothing and needs
 * nothing but the launch's inputs and outputs. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). A
 * launch that needs more than DR_SCRATCH_BYTES is refused (DR_ERANGE) before anything is enqueued. Every call on one
 * GPU shares that GPU's array (calls that overlap in time on one GPU race: keep them on one stream). The launch's
 * stream must belong to the current device (else DR_EINVAL). The first call that needs the array on a device clears
 * its counters with a fill on a stream of the library's own and waits for it before returning, so that call must not
 * be made under stream capture (refused with DR_EINVAL, nothing enqueued): a caller that captures makes one eager call
 * first; later calls enqueue only the matmul and can be captured. */
int dr_matmul_noalloc(const dr_launch* launch);
int64_t dr_scratch_bytes(void);

/* The best k_out of records [n_records][2 * rows * k] (as dr_topk writes them) per row: vals [rows][k_out] fp32
 * (-inf empty), ids [rows][k_out] int32 (-1 empty), highest first, ties to the lower id. rows <= 32 (a record's, as
 * dr_topk's), k_out <= 64. Many records
 * are merged by several workgroups a row that meet in the workspace (dr_topk_merge_workspace_bytes; zeroed once by
 * the caller; every merge leaves its counters at zero, at the same place whatever its shape, so merges and head picks
 * of any shape can share one, not overlapping in time). */
int64_t dr_topk_merge_workspace_bytes(int n_records, int rows, int k);
int dr_topk_merge(const void* records, int n_records, int rows, int k, int fp32, int k_out, float* vals,
                  int32_t* ids, void* workspace, int64_t workspace_bytes, void* stream);

/* The work split for K and M: chunks (waves per output tile, each a K range of kch values) and the rows a pass
 * takes (M picks the kernel: the GEMV for 1-2 rows, the MFMA kernel from 3, whose chunks are 256 k up to K = 3072
 * against the GEMV's up to 2048). For inspection of block-float and bf16 weights (an int4 weight runs the GEMV at any
 * M; dr_launch_plan gives any launch's own plan); results depend only on what this returns. */
int dr_plan(int k, int m, int32_t* chunks, int32_t* kch, int32_t* rows_per_pass);

/* What dr_matmul would launch for this launch, for inspection (replaces the plan dict that dense_reader/linear.py:
 * 455-495 choose/plan return): the kernel, the output tile width, the work split and the top-k records it writes. */
typedef struct dr_launch_info {
    int32_t kernel;        /* 0: the VALU GEMV (rows <= 2 a pass, and int4), 1: the MFMA kernel */
    int32_t rows_per_pass;
    int32_t tile_cols;     /* output columns of a work tile: 16 (one panel) or 32 */
    int32_t tiles;         /* work tiles of the launch */
    int32_t chunks;        /* K chunks a tile, kch values each */
    int32_t kch;
    int32_t splits;        /* workgroups a tile (split K), 1 if unsplit */
    int32_t workgroups;    /* workgroups of one pass */
    int32_t passes;        /* launches (row passes) */
    int32_t records;       /* top-k records the launch writes (0: no top-k) */
    int32_t tiles_per_record;
    int32_t waves;         /* wavefronts a workgroup (each walks its K chunks in turn) */
    int32_t tiles_per_workgroup; /* 2: a 32-row launch of more tiles than CUs, its block-float segments' tiles in
                                    pairs (bf16 segments one a workgroup), else 1 */
    int32_t lds_bytes;     /* LDS a workgroup of the first pass's kernel, static and dynamic (0 without a device) */
    int32_t reserved[2];
} dr_launch_info;
int dr_launch_plan(const dr_launch* launch, dr_launch_info* info);

/* Each workgroup of one pass of the launch (info.workgroups of them): five int32 a workgroup, (block, first tile of
 * the block, tiles, K split, first output column), tiles being 16 or 32 columns (info.tile_cols), the block the
 * caller's index in seg[]. DR_ERANGE if max_workgroups is smaller. The MI355X counterpart of the `work` list of the
 * reference's plan (dense_reader/linear.py:355-366: each core's bank, pitch, columns and first output tile). */
int dr_launch_work(const dr_launch* launch, int32_t* work, int max_workgroups);

/* A plain streaming read of `bytes` (a multiple of 16, 16-byte aligned) at p with every CU: the read ceiling the
 * matmul's weight bandwidth is measured against (bench.py --read-probe). No counterpart in the reference (a
 * measurement aid); nothing is written but, never in practice, one word of sink. */
int dr_stream_read(const void* p, int64_t bytes, uint32_t* sink, void* stream);

const char* dr_status_string(int status);
int dr_version(void);

#ifdef __cplusplus
}
#endif

#endif
