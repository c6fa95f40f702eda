/*
 * ffn_mi355x.h -- C ABI of the MI355X (gfx950) fused FFN operator
 *
 *     Y = GELU(X . W1^T) . W2^T        X [mp,kp], W1 [hp,kp], W2 [np,hp]
 *
 * Every buffer is a device pointer to a row-major, K-contiguous matrix that the
 * caller has already contiguised and zero-padded (M/H/N to 64, K to 16), exactly
 * as ops/host/inputs.py:74-90 stores them in the reference.  The library never
 * allocates or frees device memory, never synchronises the host, and enqueues
 * all work on the HIP stream it is given, so it is stream-ordered like the
 * single artifact launch it replaces (ops/api.py:37-45).
 *
 * Return codes are 0 on success or one of the negative FFN_MI355X_E* values;
 * ffn_mi355x_last_error() gives the message of the last failure on the calling
 * thread.  The Python host maps them onto the reference's exception taxonomy
 * (ops/api.py:9-14, ops/host/dispatch.py:22-39).
 */
#ifndef FFN_MI355X_H
#define FFN_MI355X_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element type of X, W1, W2, hidden and the output */
#define FFN_MI355X_FP16 0
#define FFN_MI355X_BF16 1

/* down-projection implementation (ops/host/dispatch.py:15 DOWN_IMPLS) */
#define FFN_MI355X_DOWN_BASIC 0
#define FFN_MI355X_DOWN_STREAMK 1
#define FFN_MI355X_DOWN_FULL_LOAD_A 2 /* reported unavailable, no fallback */
#define FFN_MI355X_DOWN_FULL_LOAD_B 3 /* reported unavailable, no fallback */

/* Activation of the up-projection epilogue.  The reference computes the GELU forms only; SiLU
 * and SwiGLU are the other two paths of the EagleFFN operator its analysis describes
 * (spec/MindIE-SD EagleFFN算子实现分析.md:17-71). */
#define FFN_MI355X_GELU_ERF 0      /* 0.5*z*(1+erf(z/sqrt2)), F.gelu(approximate='none') */
#define FFN_MI355X_GELU_RATIONAL 1 /* clamp + P5/Q5 rational erf, validation/reference.py:5-13 */
#define FFN_MI355X_SILU 2          /* z/(1+exp(-z)) */
#define FFN_MI355X_SWIGLU 3        /* SiLU(gate)*up: W1 holds 2*hp rows, gate and up rows interleaved
                                      in 32-row blocks (rows 64b..64b+31 = gate rows 32b..32b+31,
                                      rows 64b+32..64b+63 = up rows 32b..32b+31), zero past h */

/* Largest operand row pitch, in elements, that ffn_mi355x_set_operands accepts: a macro tile's
 * rows are addressed with 32-bit buffer offsets, and (256 + 1) rows of this pitch in 2-byte
 * elements stay below 2^31, the offset that marks a zero-filled chunk. */
#define FFN_MI355X_MAX_PITCH 4000000

/* return codes */
#define FFN_MI355X_OK 0
#define FFN_MI355X_EINVAL (-1)          /* ValueError */
#define FFN_MI355X_ENOT_APPLICABLE (-2) /* NotApplicable(ValueError) */
#define FFN_MI355X_EUNAVAILABLE (-3)    /* DependencyUnavailable(RuntimeError) */
#define FFN_MI355X_EHIP (-4)            /* RuntimeError from the HIP runtime */
#define FFN_MI355X_EDEVICE (-5)         /* RuntimeError: not a gfx950 device */

/* Tile geometry and launch shape the library chose for one FFN.  It is the
 * counterpart of the reference's Plan/Tile (ops/host/tiling.py:11-74). */
typedef struct ffn_mi355x_plan {
    int m;                       /* logical rows of X (rows m..mp-1 are zero padding) */
    int mp, kp, hp, np;          /* padded extents the plan was made for */
    int dtype, down_impl, activation; /* FFN_MI355X_GELU_ERF .. FFN_MI355X_SWIGLU */
    int block_num;               /* persistent workgroups per launch (<= CU count) */
    int up_variant, down_variant;
    int up_bm, up_bn, up_bk;     /* up-projection macro tile (M x H x K) */
    int down_bm, down_bn, down_bk; /* down-projection macro tile (M x N x H) */
    int up_tiles, up_grid;
    int down_tiles, down_grid;   /* down_grid <= block_num: fewer for Basic when there are fewer
                                    tiles, and for Stream-K when that cuts every split tile into
                                    equal pieces */
    int down_k_iters;            /* BK-deep iterations along H per down tile */
    int down_dp_tiles;           /* tiles reduced whole by one workgroup */
    int down_sk_tiles;           /* tiles whose H-range is split over workgroups */
    int down_slots_per_wg;       /* FP32 partial-tile slots per workgroup */
    size_t workspace_bytes;      /* FP32 partial-tile slots of the Stream-K down and the split up */
    /* Operand layout.  ffn_mi355x_make_plan sets the padded buffers (k = kp, h = hp,
       n = np, ldx = ldw1 = kp, ldw2 = hp); ffn_mi355x_set_operands may point the plan at
       operands of their logical widths instead. */
    int k, h, n;                 /* logical K, H and N */
    int ldx, ldw1, ldw2;         /* row pitches, in elements, of X, W1 and W2 */
    /* Split up GEMM.  When its tiles fill at most half of block_num and it is at least 16
       iterations deep, every up tile is split along K over up_grid workgroups: FP32 partials
       in the workspace, and the last piece of each tile to finish sums them in K order,
       applies the GELU and stores hidden.  up_sk_tiles = 0: one workgroup per tile.
       workspace_bytes covers both GEMMs (they run one after the other on the stream). */
    int up_k_iters;              /* BK-deep iterations along K per up tile */
    int up_sk_tiles;             /* up tiles split along K (0 or up_tiles) */
    int up_slots_per_wg;         /* FP32 partial-tile slots per workgroup of the split up */
    /* Gathered rows of X (ffn_mi355x_set_x_rows): x_d1 = 0 reads row r at r * ldx; otherwise
       row r = (i0 * x_d1 + i1) * x_d2 + i2 starts at element i0*x_s0 + i1*x_s1 + i2*x_s2. */
    int x_d1, x_d2, x_s0, x_s1, x_s2;
    /* 1: the FFN runs as one launch (up and down tiles in one persistent grid, a down tile
       starting as soon as the hidden rows it reads are stored), where a single-launch kernel is
       compiled for the tile pair (ffn_mi355x_set_single_launch; ffn_mi355x_make_plan leaves it
       0, the two launches having measured faster); 0: two stream-ordered launches, up then
       down. */
    int single_launch;
    /* Check word over every field above, written by ffn_mi355x_make_plan and
       ffn_mi355x_set_operands.  The run entry points refuse a plan whose fields no longer
       match it (EINVAL "invalid plan"): its grids, tile counts and workspace size decide
       which memory the kernels touch, so a plan is used only as the library left it. */
    unsigned long long stamp;
} ffn_mi355x_plan;

/* Device check replacing the Ascend950/AIC checks of ops/api.py:58-66:
 * writes the CU count and gcnArchName of `device`; FFN_MI355X_EDEVICE if the
 * device is not gfx950. */
int ffn_mi355x_query(int device, int* cu_count, char* arch, int arch_len);

/* Tile selection and Stream-K schedule, host-only (no device call).  Mirrors
 * make_plan (ops/host/tiling.py:58-74): FFN_MI355X_EUNAVAILABLE for the
 * full-load down variants (ops/host/dispatch.py:61-66), FFN_MI355X_EINVAL for a
 * block_num outside [1, 65535], FFN_MI355X_ENOT_APPLICABLE for Stream-K shapes
 * with no remainder tiles or fewer than two H iterations (tiling.py:65-70).
 * up_variant / down_variant < 0 let the library choose; >= 0 forces a tile.
 * m is the logical row count: the zero-padding rows of X and hidden are then
 * never fetched (they read as zeros), which matters for small-M decode shapes. */
int ffn_mi355x_make_plan(int m, int mp, int kp, int hp, int np, int dtype, int down_impl,
                         int activation, int block_num, int up_variant, int down_variant,
                         ffn_mi355x_plan* plan);

/* Reads the operands in place at their logical widths instead of from buffers padded
 * to the plan's extents: X [m, k] with row pitch ldx, W1 [h, k] with pitch ldw1, W2 [n, h]
 * with pitch ldw2 (elements; each row 16-byte aligned, i.e. pitches and the base addresses
 * multiples of 8 elements / 16 bytes).  Columns past k and rows past h and n read as zero
 * through the kernels' range checks, and hidden columns [h, hp) are written as GELU(0) = 0.
 * k must be a multiple of 8 or equal kp; with h not a multiple of 8, W2 must span hp
 * columns (ldw2 >= hp, zero past h).  No counterpart in the reference, whose prepare step
 * always copies into padded buffers (ops/host/inputs.py:74-90).  EINVAL on a bad layout,
 * including a pitch above FFN_MI355X_MAX_PITCH. */
int ffn_mi355x_set_operands(ffn_mi355x_plan* plan, int k, int h, int n, int ldx, int ldw1, int ldw2);

/* Reads X in place as a strided view instead of rows at one pitch: the plan's m rows form a
 * [m / (d1*d2), d1, d2] grid, row (i0, i1, i2) holding k contiguous elements from element
 * i0*s0 + i1*s1 + i2*s2 of x.  This is how a permuted activation (the Canonical layout's
 * transposed view, a [B, S, D] tensor read as [S, B, D]) is consumed without the copy the
 * reference's prepare step makes (ops/host/inputs.py:74-90: x.contiguous() into [mp, kp]).
 * d1, d2 >= 1 dividing m; strides >= 0 and multiples of 8 elements (16-byte rows); the
 * furthest element read, ((m/(d1*d2)-1)*s0 + (d1-1)*s1 + (d2-1)*s2 + k) * 2 bytes from x,
 * below 2^31.  d1 = 0 restores rows at pitch ldx.  Kept by ffn_mi355x_set_operands; EINVAL
 * on a bad grid, plan unchanged. */
int ffn_mi355x_set_x_rows(ffn_mi355x_plan* plan, int d1, int d2, int s0, int s1, int s2);

/* Turns the single launch of a plan on (1) or off (0).  On needs a compiled single-launch kernel
 * for the plan's tile pair, a Basic down, an unsplit up GEMM with the GELU epilogue, at least
 * eight up tile rows (one per XCD) and a K of at most 8192: ENOT_APPLICABLE otherwise.  A plan
 * that can run as one launch holds at least the workspace's counter region in workspace_bytes
 * either way, so its workspace serves both forms.  An X read as gathered rows
 * (ffn_mi355x_set_x_rows) runs as two launches whatever the setting.  No counterpart in the
 * reference, whose FFN is always one artifact (ops/api.py:43). */
int ffn_mi355x_set_single_launch(ffn_mi355x_plan* plan, int on);

/* Workspace bytes a plan needs (0 for the Basic down without a split up GEMM or a single
 * launch). */
int ffn_mi355x_workspace_bytes(const ffn_mi355x_plan* plan, size_t* bytes);

/* Bytes at the start of every workspace that hold the split tiles' arrival counters (one
 * 32-bit counter per split tile and wave: the Stream-K down's from the start of the region, a
 * split up GEMM's from its end; each split tile's counters start FFN_MI355X_SPLIT_COUNTER_WORDS
 * words after the previous tile's when both GEMMs' split tiles fit the region that way, else
 * they are packed, one word per wave of the tile).  Each GEMM's launch clears the other's counters before any
 * tile, and every launch leaves its own zero: a Stream-K down therefore always starts from zero
 * counters when its up GEMM ran first in the same call (ffn_mi355x_run, or ffn_mi355x_up given
 * the workspace), whatever the region held, and a split up GEMM from its second call on.  Zero
 * the region before the first call of a plan with a split up GEMM (e.g. allocate the workspace
 * zero-filled).  A workspace can then serve any plans whose workspace_bytes it covers, one call
 * after another; calls that overlap on one workspace race.  The rest of the workspace needs no
 * initialisation.  No counterpart in the reference, whose Stream-K reduction is a separate
 * phase (ops/kernel/ffn.py:1035-1175). */
#define FFN_MI355X_WORKSPACE_COUNTER_BYTES (64u << 10)
/* Words from one split tile's arrival counters to the next (a 128-byte line each). */
#define FFN_MI355X_SPLIT_COUNTER_WORDS 32

/* FFN_MI355X_WORKSPACE_COUNTER_BYTES when the plan needs a workspace, else 0. */
int ffn_mi355x_workspace_counter_bytes(const ffn_mi355x_plan* plan, size_t* bytes);

/* The whole FFN: up GEMM + GELU epilogue writing `hidden` [mp,hp] in the input
 * dtype, then the Basic or Stream-K down GEMM writing `out` [mp,np].  Replaces
 * the single artifact(*tensors, block_num) launch of ops/api.py:43 built by
 * compile_kernel (ops/host/dispatch.py:97-116) from ops/kernel/ffn.py.
 * `ws` must hold plan->workspace_bytes whenever that is nonzero (Stream-K down or
 * split up), its counter bytes as FFN_MI355X_WORKSPACE_COUNTER_BYTES describes; it may be
 * NULL otherwise.
 * The Stream-K down is one launch: the pieces of a split tile store FP32 partial tiles to `ws`,
 * and the last piece to arrive sums them in ascending K order, rounds once and stores the tile.
 * A split up is the same with the GELU applied after the sum. */
int ffn_mi355x_run(const ffn_mi355x_plan* plan, const void* x, const void* w1,
                   const void* w2, void* hidden, void* out, void* ws, void* hip_stream);

/* Bytes of device scratch behind ffn_mi355x_run_noalloc (per GPU, held until the process ends). */
#define FFN_MI355X_NOALLOC_SCRATCH_BYTES (32u << 20)

/* ffn_mi355x_run for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The Stream-K partial tiles (and those of a split up GEMM) go to a scratch array of the
 * library itself, FFN_MI355X_NOALLOC_SCRATCH_BYTES per GPU; the caller passes the operands,
 * hidden and out as for ffn_mi355x_run, and no workspace.  A plan whose workspace_bytes exceeds
 * the scratch is refused with FFN_MI355X_EINVAL before any launch.  The call allocates and
 * frees nothing.  Every call on one GPU shares that GPU's scratch: calls that overlap on one GPU
 * (on different streams, or from different threads) race and must be serialised by the caller.
 * The scratch starts zero-filled and every call leaves its arrival counters zero again; every
 * partial is written before it is read within a call, so nothing needs clearing. */
int ffn_mi355x_run_noalloc(const ffn_mi355x_plan* plan, const void* x, const void* w1,
                           const void* w2, void* hidden, void* out, void* hip_stream);

/* ffn_mi355x_run with per-column biases, the EagleFFN form
 *     Y = act(X . W1^T + b1) . W2^T + b2
 * (spec/MindIE-SD EagleFFN算子实现分析.md:17-40; the reference operator has no bias).
 * b1 holds h values (SwiGLU: 2*hp, interleaved like W1's rows), b2 holds n values, in the
 * storage type; each is added in FP32 before the activation (b1) or the cast (b2).  Both or
 * neither (FFN_MI355X_EINVAL otherwise); NULL, NULL is ffn_mi355x_run. */
int ffn_mi355x_run_ex(const ffn_mi355x_plan* plan, const void* x, const void* w1, const void* b1,
                      const void* w2, const void* b2, void* hidden, void* out, void* ws,
                      void* hip_stream);

/* The two stages of ffn_mi355x_run_ex alone (b1 / b2 may be NULL: no bias). */
int ffn_mi355x_up_ex(const ffn_mi355x_plan* plan, const void* x, const void* w1, const void* b1,
                     void* hidden, void* ws, void* hip_stream);
int ffn_mi355x_down_ex(const ffn_mi355x_plan* plan, const void* hidden, const void* w2,
                       const void* b2, void* out, void* ws, void* hip_stream);

/* Stage 1 alone: up-projection with GELU epilogue (ops/kernel/ffn.py:207-360,
 * 540-581, the cube/vector up regions of both kernels).  `ws` holds
 * plan->workspace_bytes, counters zero, when plan->up_sk_tiles > 0 (split up); it may be NULL
 * otherwise. */
int ffn_mi355x_up(const ffn_mi355x_plan* plan, const void* x, const void* w1,
                  void* hidden, void* ws, void* hip_stream);

/* Stage 2 alone: Basic (ops/kernel/ffn.py:377-529) or Stream-K
 * (ops/kernel/ffn.py:951-1423) down-projection. */
int ffn_mi355x_down(const ffn_mi355x_plan* plan, const void* hidden, const void* w2,
                    void* out, void* ws, void* hip_stream);

/* Number of tile variants compiled in, and the geometry of one of them. */
int ffn_mi355x_num_variants(void);
int ffn_mi355x_variant_info(int variant, int* bm, int* bn, int* bk, int* waves, int* stages,
                            int* lds_bytes);

/* Waves of a tile variant that only refill its LDS stages (0 for most tiles; `waves` above
 * counts them too), or a negative code for a variant out of range.  No counterpart in the
 * reference, whose tiles are fixed (ops/host/tiling.py:11-25): it describes the library's
 * tile table for planners and tests. */
int ffn_mi355x_variant_refill_waves(int variant);

/* MFMA block edge of a tile variant: 32 (v_mfma_f32_32x32x16) or 16 (v_mfma_f32_16x16x32), or a
 * negative code for a variant out of range.  No counterpart in the reference (its tiles are
 * fixed, ops/host/tiling.py:11-25): tiles of the two edges sum each output in a different
 * order, so only tiles of one edge compute bit-identical results. */
int ffn_mi355x_variant_mfma_edge(int variant);

/* Message of the last failure on this thread ("" if none). */
const char* ffn_mi355x_last_error(void);

/* Text of a return code. */
const char* ffn_mi355x_strerror(int code);

/* Library build tag (target architecture and source revision). */
const char* ffn_mi355x_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FFN_MI355X_H */
