/*
 * ftk.h -- C ABI of the MI355X (gfx950) skinny BF16 projection library, libftk.so.
 *
 * The reference (john-jpet/fast-transformer) has no C ABI: its path is Python
 * functions over Triton kernels (the .py files of engine/kernels/). Each entry point below
 * replaces the device work under one of those functions; the Python package
 * `kernels` (fast-transformer_amd/kernels/) keeps the reference's signatures and
 * calls these through ctypes.
 *
 * Conventions
 *   - Tensors are plain device pointers. BF16 is passed as raw 16-bit patterns.
 *     Matrices are row-major: x[M, K], W[N, K] (PyTorch Linear layout, K
 *     contiguous), y[M, N]. y = x @ W^T with FP32 accumulation and one
 *     round-to-nearest-even to BF16 (engine/kernels/linear.py:1-6).
 *   - `stream` is a hipStream_t (NULL = the null stream). Work is only
 *     enqueued: nothing synchronizes, nothing allocates, so every entry point
 *     can be captured into a hipGraph.
 *   - Return value: FTK_OK or an ftk_status code. Nothing is launched when a
 *     code other than FTK_OK or FTK_ERR_HIP is returned.
 *   - M (rows of x) is 1..FTK_MAX_ROWS, as the reference's MAX_ROWS = 32
 *     (engine/kernels/linear.py:343); larger M is the caller's native GEMM.
 *   - Workspaces hold per-call scratch (RMSNorm row scales, per-workgroup
 *     argmax keys, a tile-claim counter). Zero a workspace once when it is
 *     allocated: the argmax key words (from byte 256) and the claim counter
 *     (bytes 128..131) must be zero when a call starts, and every call leaves
 *     them zero again (the one-launch argmax reads a non-zero word as a key of
 *     the current call; the counter's last claim puts it back). Nothing else
 *     carries over between calls. Calls that share a workspace must not run
 *     concurrently. (The norm's row sums of ftk_rows.sumsq_out / sumsq are the
 *     caller's own buffer, written by one call for a later one to read.)
 *   - No kernel uses device-scope fences. The RING kind's long walks (lm_head
 *     + argmax with the norm prologue, 1..16 rows) claim their last tiles with
 *     agent-scope atomic adds on the workspace's counter; a workspace smaller
 *     than ftk_project_workspace_bytes() (or none, where no argmax needs one)
 *     keeps those walks in their static order. One workgroup waits on others:
 *     the extra, last workgroup of a one-launch lm_head + argmax (the STREAM
 *     kind at M = 1, the default where the RING kind's claimed tail does not
 *     apply) reads the other workgroups' key words, with a bounded wait (1 s;
 *     then the row's id is -1). The others never wait, so its wait ends in
 *     whatever order the workgroups run. After an id of -1 the workspace may
 *     hold that call's late key words: zero it again before the next call.
 */
#ifndef FTK_H
#define FTK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FTK_MAX_ROWS 32

typedef enum ftk_status {
  FTK_OK = 0,
  FTK_ERR_INVALID = 1,      /* null pointer, non-positive size, M > FTK_MAX_ROWS, bad flag */
  FTK_ERR_UNSUPPORTED = 2,  /* shape/alignment this fused entry point does not take (K % 8, 16-byte alignment) */
  FTK_ERR_WORKSPACE = 3,    /* workspace missing or smaller than *_workspace_bytes() */
  FTK_ERR_HIP = 4,          /* the HIP launch failed; see ftk_last_hip_error() */
  FTK_ERR_TOO_LARGE = 5     /* the call needs more scratch than FTK_STATIC_SCRATCH_BYTES
                               (ftk_lm_head_argmax_static_bf16) */
} ftk_status;

/* Bytes of the static device scratch array of ftk_lm_head_argmax_static_bf16 (one per GPU). */
#define FTK_STATIC_SCRATCH_BYTES (1 << 20)

typedef enum ftk_epilogue {
  FTK_EPI_STORE = 0,   /* y[m, n] = bf16(sum) */
  FTK_EPI_SWIGLU = 1,  /* y[m, j] = bf16(bf16(silu(bf16(g_j))) * bf16(u_j)), W = cat(W_gate, W_up) */
  FTK_EPI_ARGMAX = 2   /* logits (optional) + lowest-index greedy id per row */
} ftk_epilogue;

/* OR-ed into the epilogue argument of ftk_plan_project / ftk_project_workspace_bytes:
 * plan a call that has the RMSNorm prologue (gamma != NULL). Some launch shapes
 * exist only without it, so the plan (and the workspace size) can differ. */
#define FTK_PLAN_PROLOGUE 0x100
/* OR-ed in as well: the call's prologue adds a residual (ftk_rows.residual). The RING kind
 * does not take that add, so such a call is planned without it. */
#define FTK_PLAN_RESIDUAL 0x200

typedef enum ftk_kind {
  FTK_KIND_AUTO = 0,
  FTK_KIND_GEMV = 1,     /* M <= 4: HBM-streaming GEMV (v_dot2_f32_bf16, LDS-resident x) */
  FTK_KIND_MFMA = 2,     /* M >= 4: v_mfma_f32_16x16x32_bf16 tiles */
  FTK_KIND_GENERIC = 3,  /* any shape/alignment, scalar loads; store epilogue only */
  FTK_KIND_STREAM = 4,   /* M <= 8, K = 512 C KW: HBM-streaming GEMV, x slice in registers,
                            rolling weight prefetch, one barrier per workgroup */
  FTK_KIND_MFMA_STREAM = 5, /* M <= 16, K = 32 S KW: the STREAM schedule on 16x16x32 MFMA tiles */
  FTK_KIND_QUAD = 6,        /* M <= 16, K = 128 C KW: the STREAM schedule on 16-block 4x4x4 MFMAs,
                               weights loaded as 4 rows x 256 contiguous bytes per wave load */
  FTK_KIND_STAGE = 7,       /* M <= 16, K = 128 C KW: QUAD's weight loads staged through LDS into
                               16x16x32 MFMA tiles */
  FTK_KIND_RING = 8         /* M = 1..16, K = 128 C KW: weight and x segments loaded straight into a
                               per-wave LDS ring (global_load_lds_dwordx4), 16x16x32 MFMA tiles;
                               no residual-add prologue */
} ftk_kind;

/* Launch choice for one projection (the reference's per-shape config tuple,
 * engine/kernels/linear.py:179 `kind, block_n, block_k, splits, warps`).
 * Zero fields mean "planner default". */
typedef struct ftk_config {
  int kind;            /* ftk_kind */
  int rows_per_wave;   /* GEMV, STREAM: weight rows per row group per tile (1..8);
                          MFMA: rows per workgroup (16, 32, 64); MFMA_STREAM, STAGE: rows per tile
                          (16, 32); QUAD: weight rows per row group per tile (4, 8, 16, 24; SwiGLU
                          8, 16, 24); RING: 16 (SwiGLU: 8 gate + 8 up rows), or for the
                          STORE epilogue 12 (at K = 4096), or 24 (at up to 8 rows) */
  int unroll;          /* GEMV: 16-byte chunks per lane per load batch (1, 2, 4);
                          MFMA: K steps of loads in flight per wave (T = 1, 2: 4 or 8; T = 4: 2 or 4);
                          STREAM, QUAD: unused (K fixes the chunks per lane);
                          MFMA_STREAM: K steps of weight loads in flight per wave (2, 4, 8);
                          STAGE: 128-wide K segments of weight loads in flight per wave (2..6);
                          RING: units (K segments of a tile) in flight per wave (2; 3 at K = 12288) */
  int groups_per_cu;   /* GEMV, STREAM, MFMA_STREAM, QUAD, STAGE, RING: grid cap = groups_per_cu * CUs (grid-stride
                          beyond; the STREAM kinds raise the grid so no workgroup walks more tiles
                          than its LDS holds); MFMA: unused */
  int waves;           /* MFMA, MFMA_STREAM, STAGE, RING: waves per workgroup splitting K (4, 8, 16);
                          GEMV, STREAM: waves per row group splitting K (1, 2, 4, 8; a workgroup is
                          4 waves, or 8 when 8 split K);
                          QUAD: waves per row group splitting K (4, 8, 16; the workgroup is
                          max(4, waves) waves) */
} ftk_config;

typedef struct ftk_plan {
  int kind;
  int rows_per_wave;
  int unroll;
  int waves;                /* MFMA: waves per workgroup; GEMV: waves per row group */
  int grid;                 /* workgroups launched */
  int tiles;                /* row tiles (GEMV: walked grid-stride; MFMA: 64 rows each) */
  int threads;              /* threads per workgroup (64 per wave) */
  int64_t lds_bytes;        /* dynamic LDS per workgroup */
  int splits;               /* K slices per output (always 1: no split-K across workgroups) */
  int k_slice;              /* K elements per slice (= K) */
  int64_t workspace_bytes;  /* workspace this launch needs (0 = none) */
} ftk_plan;

/* ---- library ------------------------------------------------------------- */
const char* ftk_version(void);
const char* ftk_status_string(int status);
int ftk_last_hip_error(void);          /* hipError_t of the last FTK_ERR_HIP on this thread */
int ftk_device_compute_units(void);    /* CUs of the current device, or -1 without a device */
/* Workgroups of a persistent launch over `tiles` tiles on `units` compute units: the fewest
 * that keep every workgroup's walk at ceil(tiles / units) tiles (engine/kernels/gemm.py:330-338
 * persistent_programs). The planner sizes the STREAM, QUAD, STAGE and MFMA_STREAM grids with it.
 * 0 when tiles or units is not positive. Host only. */
int ftk_persistent_programs(int tiles, int units);
/* Tile that step `step` of RING workgroup `wg` computes in a grid of `grid` over `tiles` tiles
 * (the workgroup runs steps 0 .. ceil((tiles - wg) / grid) - 1). In every full round of `grid`
 * tiles the workgroups of one XCD (wg % 8) take one contiguous run; otherwise wg + step * grid.
 * No counterpart in the reference (its persistent kernels take tile pid + i * programs); exported
 * so the mapping can be checked on the host. -1 for a step the workgroup does not run. Host only. */
int ftk_ring_tile(int wg, int step, int grid, int tiles);

/* ---- projections ------------------------------------------------------------ */

/* y = x @ W^T.  Replaces the device work of linear(x, weight, split_ok)
 * (engine/kernels/linear.py:489-523) and _project (linear.py:178-314).
 * Any N, K and alignment (unaligned or K % 8 != 0 takes the generic kind). */
int ftk_linear_bf16(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K, void* stream);

/* y = rms_norm(x, gamma, eps) @ W^T with the norm folded into the projection's
 * prologue. Replaces rms_norm (engine/kernels/rmsnorm.py:49-72, cast order
 * :35-46) followed by linear (layers.py:44 QKV). Needs K % 8 == 0, 16-byte
 * aligned x, W, gamma (else FTK_ERR_UNSUPPORTED). */
int ftk_rms_norm_linear_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M,
                             int64_t N, int64_t K, void* stream);

/* y[M, I] = swiglu(xn @ W^T) with W = cat(W_gate, W_up) [2I, K] and
 * xn = rms_norm(x) when gamma != NULL (else x). Replaces linear(gate_up) +
 * swiglu (engine/layers.py:99-102, engine/kernels/swiglu.py:13-40). */
int ftk_gate_up_swiglu_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M,
                            int64_t I, int64_t K, void* stream);

/* Greedy ids of xn @ W^T (xn = rms_norm(x) when gamma != NULL), lowest index
 * on ties of the BF16-rounded logits; logits [M, V] written when non-NULL,
 * top[M] = winning logit (FP32) when non-NULL; ids are int32 (ids_bytes 4) or
 * int64 (8). Replaces the final norm + lm_head linear + argmax
 * (engine/decode.py:274-278, engine/kernels/argmax.py:51-70, fused_argmax
 * argmax.py:112-129, greedy_tokens argmax.py:132-167). */
int ftk_lm_head_argmax_bf16(const void* x, const void* gamma, float eps, const void* w, void* logits, void* ids,
                            int ids_bytes, float* top, int64_t M, int64_t V, int64_t K, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* ftk_lm_head_argmax_bf16 for callers that cannot allocate device memory: code under
 * graph capture that may not call hipMalloc, tight serving loops, harnesses that forbid
 * allocation. No counterpart in the reference. It takes no workspace and allocates nothing:
 * the per-workgroup argmax keys live in a static device array of FTK_STATIC_SCRATCH_BYTES
 * (1 MiB) that every GPU the library runs on holds until the process ends. The array starts
 * zeroed and every call leaves its key words zero, as the workspace convention above asks.
 * Results are those of ftk_lm_head_argmax_bf16 bit for bit (same kernels). A call that needs
 * more keys than the array
 * holds (e.g. 32 rows of a 151936-entry vocabulary) returns FTK_ERR_TOO_LARGE and launches nothing.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, two
 * threads) race and give wrong ids; keep them in one stream. */
int ftk_lm_head_argmax_static_bf16(const void* x, const void* gamma, float eps, const void* w, void* logits,
                                   void* ids, int ids_bytes, float* top, int64_t M, int64_t V, int64_t K,
                                   void* stream);

/* Workspace bytes ftk_project_bf16 needs for this shape on the current device:
 * per-workgroup argmax keys (FTK_EPI_ARGMAX) and the RMSNorm row scales of the
 * MFMA kind (gamma != NULL). Other calls need none (NULL is fine). OR
 * FTK_PLAN_PROLOGUE into `epilogue` for a call with gamma. */
int64_t ftk_project_workspace_bytes(int64_t M, int64_t N, int64_t K, int epilogue, const ftk_config* cfg);

/* General form of the three above with an explicit launch choice (cfg may be
 * NULL): the tuner's entry point (engine/kernels/linear.py:436-481 _choose). */
int ftk_project_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M, int64_t N,
                     int64_t K, int epilogue, void* ids, int ids_bytes, float* top, void* workspace,
                     int64_t workspace_bytes, const ftk_config* cfg, void* stream);

/* The prologue's input rows beyond a plain x: the residual side of the norm
 * (engine/kernels/rmsnorm.py:75-125 add_rms_norm, called at engine/decode.py:240-261)
 * and the embedding gather of the first layer (rmsnorm.py:128-162 embed_rms_norm,
 * decode.py:229). The norm then reads s[m] = bf16(xrow(m) + residual[m]) (no add
 * without a residual), xrow(m) = x[x_ids[m]] (x a [rows, K] table) or x[m], and
 * s is stored into `sum` when non-NULL: the BF16 residual stream the next layer
 * adds to. `sum` must not overlap x, residual or y. */
typedef struct ftk_rows {
  const void* residual;  /* [M, K] BF16, or NULL */
  void* sum;             /* [M, K] BF16 out, or NULL */
  const void* x_ids;     /* [M] row indices into x, or NULL */
  int x_ids_bytes;       /* 4 (int32) or 8 (int64) */
  int64_t x_rows;        /* rows of the table x (required, >= 1, with x_ids). The ids live on the
                            device, so the device clamps them into the table: an id below 0 reads
                            row 0 and an id at or past x_rows reads row x_rows - 1 */
  /* The norm's statistics carried from the projection that writes a row stream to the
   * norm that reads it (the RING kind, M = 1..16). No counterpart in the reference,
   * whose norm reads its input rows (engine/kernels/rmsnorm.py:21-46).
   * sumsq_out: [M, ceil(N / 16)] FP32 out (STORE epilogue, 16-row tiles): element
   *   [m, t] is the sum of the squares of the BF16 outputs y[m, 16 t .. 16 t + 15]
   *   as stored (after the residual add of ftk_project_add_rows_bf16).
   * sumsq: [M, K / 16] FP32 in (needs gamma; no residual, sum or x_ids): those sums
   *   for x, as a call with sumsq_out wrote them; the prologue sums them (in a fixed
   *   order) instead of reading x's rows. They must describe this x: nothing checks.
   * Either one on a launch that is not RING (or sumsq_out not 16-row STORE) returns
   * FTK_ERR_UNSUPPORTED. */
  const float* sumsq;
  float* sumsq_out;
} ftk_rows;

/* ftk_project_bf16 with the prologue's rows described by `rows` (NULL: x as is).
 * Needs gamma. Kinds without the fused form return FTK_ERR_UNSUPPORTED (the
 * generic kind; the MFMA kind when sum is NULL). */
int ftk_project_rows_bf16(const void* x, const ftk_rows* rows, const void* gamma, float eps, const void* w, void* y,
                          int64_t M, int64_t N, int64_t K, int epilogue, void* ids, int ids_bytes, float* top,
                          void* workspace, int64_t workspace_bytes, const ftk_config* cfg, void* stream);

/* y = bf16( f32(bf16(x @ w^T)) + f32(residual) ), [M, N]: the projection whose
 * output joins the residual stream, with the add of add_rms_norm
 * (engine/kernels/rmsnorm.py:86-95) moved into its epilogue. At the reference's
 * call sites (engine/decode.py:236-243 and :258-261, the O and down projections
 * of engine/layers.py:86 and :101-102 followed by add_rms_norm) the stored value
 * is exactly add_rms_norm's `summed` output, so the next norm can read it as a
 * plain x (ftk_rms_norm_linear_bf16 and friends) and no prologue reads the
 * residual again. `y` may be `residual` itself (in place); no other overlap.
 * No reference counterpart as one call: it fuses linear.py:489-523 with the add
 * of rmsnorm.py:98-125. cfg may be NULL. */
int ftk_project_add_bf16(const void* x, const void* w, const void* residual, void* y, int64_t M, int64_t N,
                         int64_t K, const ftk_config* cfg, void* stream);

/* ftk_project_add_bf16 that also writes rows->sumsq_out (the only field it takes; rows may be
 * NULL): the residual stream's sums of squares for the norm that reads it next. Returns
 * FTK_ERR_UNSUPPORTED, launching nothing, where the launch is not a 16-row RING tile. */
int ftk_project_add_rows_bf16(const void* x, const ftk_rows* rows, const void* w, const void* residual, void* y,
                              int64_t M, int64_t N, int64_t K, const ftk_config* cfg, void* stream);

/* ---- standalone operators ---------------------------------------------------- */

/* rms_norm(x, weight, eps) (engine/kernels/rmsnorm.py:49-72): x rows of
 * `row_stride` elements, y contiguous [rows, cols]. */
int ftk_rms_norm_bf16(const void* x, int64_t row_stride, const void* gamma, void* y, int64_t rows, int64_t cols,
                      float eps, void* stream);

/* add_rms_norm(x, residual, weight, eps) (engine/kernels/rmsnorm.py:98-125):
 * x is BF16 [rows, cols] (x_splits = 0) or the FP32 partials of a Split
 * [x_splits, rows*cols] with split stride x_split_stride elements
 * (engine/kernels/merged.py:13-45). Writes y (normalized) and sum (BF16 x + r). */
int ftk_add_rms_norm_bf16(const void* x, int x_splits, int64_t x_split_stride, const void* residual,
                          const void* gamma, void* y, void* sum, int64_t rows, int64_t cols, float eps, void* stream);

/* embed_rms_norm(token_ids, table, weight, eps) (engine/kernels/rmsnorm.py:145-162):
 * hidden[r] = table[ids[r]] (the residual stream), y[r] = rms_norm(hidden[r]).
 * Precondition: every id lies in [0, table rows). The table's row count is not an
 * argument (the reference's signature), so ids are not checked; callers that cannot
 * promise valid ids use ftk_project_rows_bf16, whose gather clamps them. */
int ftk_embed_rms_norm_bf16(const void* ids, int ids_bytes, const void* table, const void* gamma, void* y,
                            void* hidden, int64_t rows, int64_t cols, float eps, void* stream);

/* swiglu(packed) (engine/kernels/swiglu.py:27-40): packed [rows, 2*width] BF16
 * (splits = 0) or FP32 split partials; out [rows, width]. */
int ftk_swiglu_bf16(const void* packed, int splits, int64_t split_stride, void* out, int64_t rows, int64_t width,
                    void* stream);

/* argmax(logits, top=) (engine/kernels/argmax.py:51-70): BF16 logits [rows, vocab]. */
int ftk_argmax_bf16(const void* logits, int64_t rows, int64_t vocab, void* ids, int ids_bytes, float* top,
                    void* workspace, int64_t workspace_bytes, void* stream);

/* bf16(sum of FP32 split partials) (engine/kernels/linear.py:81-93 _merge_projection). */
int ftk_merge_splits_bf16(const float* partial, int64_t splits, int64_t count, void* out, void* stream);

/* Workspace bytes of ftk_argmax_bf16 for `rows` rows of `vocab` logits. */
int64_t ftk_argmax_workspace_bytes(int64_t rows, int64_t vocab);

/* ---- decode attention ------------------------------------------------------------ */
/* Launch choice of the split-KV decode attention (the reference's layout tuple
 * `block_n, splits, warps`, engine/kernels/decode_attention.py:152-157).
 * Zero fields mean "planner default". */
typedef enum ftk_attn_kind {
  FTK_ATTN_AUTO = 0,
  FTK_ATTN_ROWS = 1,  /* any D in {64, 128}, up to 8 query heads per KV head: v_dot2 scores summed
                         over each cache row's lanes, an online softmax per lane, p V on the VALU */
  FTK_ATTN_QUAD = 2   /* D = 128, up to 4 query heads per KV head: scores on 16-block 4x4x4 MFMAs fed
                         by 4 cache rows x 256 bytes per wave load, one softmax step per (row, head),
                         p V on the VALU */
} ftk_attn_kind;
typedef struct ftk_attn_config {
  int kind;    /* ftk_attn_kind */
  int splits;  /* slot intervals per (row, KV head), at most 1024; 1 = no merge launch */
  int waves;   /* waves per workgroup (4, 8) */
  int unroll;  /* ROWS: cache rows of K (and of V) in flight per lane per step (2, 4, 8);
                  QUAD: groups of 16 cache rows per wave step, the loads of the next step in flight (1, 2) */
} ftk_attn_config;
typedef struct ftk_attn_plan {
  int kind;
  int splits;               /* slot intervals per (row, KV head) */
  int chunk;                /* slots per interval */
  int waves;
  int unroll;
  int grid;                 /* partials workgroups: rows * KV heads * splits */
  int64_t workspace_bytes;  /* FP32 partials + (max, denominator) pairs; 0 when splits = 1 */
} ftk_attn_plan;
/* out = softmax(q k^T * scale) v over the cache slots 0..position of each row,
 * for a one-token decode query: q [B, Hq, D] (the reference's [B, Hq, 1, D]),
 * k, v [B, Hkv, C, D], out [B, Hq, D] (the reference's [B, 1, Hq, D]); BF16.
 * Query head h reads KV head h / (Hq / Hkv). `position` is int64: one slot
 * index for every row (positions = 1, the reference's [1] tensor) or one per
 * row (positions = B). Slots past min(position, C - 1) are never read into
 * the result (they may hold NaN). Scores and sums are FP32; p is rounded to
 * BF16 before it weights V. D is 64 or 128; Hq / Hkv <= 8; q, k, v, out
 * 16-byte aligned. Replaces decode_attention and its kernels
 * (engine/kernels/decode_attention.py:31-149, :229-258). */
int ftk_decode_attention_bf16(const void* q, const void* k, const void* v, const int64_t* position, int positions,
                              void* out, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity,
                              int64_t dim, double scale, void* workspace, int64_t workspace_bytes,
                              const ftk_attn_config* cfg, void* stream);
/* One-token decode attention that starts from the packed QKV rows: the Q/K head
 * norm + RoPE + cache update of ftk_qk_rope_cache_bf16 (decode form: whole
 * cos/sin tables [table_rows, D], row b rotates at position + phases[b], phases
 * null = 0) runs in the attention kernel's prologue, then the attention of
 * ftk_decode_attention_bf16 over slots 0..position. packed [B, (Hq + 2 Hkv) D]
 * BF16; the key and value heads go to keys / values [B, Hkv, C, D] at slot
 * position (when it lies in the cache), out [B, Hq, D]. Arithmetic and roundings
 * are those of the two entry points; the order of FP32 sums differs, so results
 * agree with the two-launch form within a BF16 ulp, not bit for bit. A phase
 * outside the tables leaves that row's output unspecified and its slot
 * unwritten. QUAD kind only: D = 128, Hq / Hkv <= 4, every pointer 16-byte
 * aligned (else FTK_ERR_UNSUPPORTED, and the caller takes the two launches). The
 * workspace is that of ftk_decode_attention_bf16 for the same shape and cfg.
 * Replaces qk_rope_cache + decode_attention of a one-token decode step
 * (engine/layers.py:51-55, :76; engine/kernels/qk_rope.py:97-129,
 * engine/kernels/decode_attention.py:229-258). */
int ftk_rope_decode_attention_bf16(const void* packed, const void* q_gain, const void* k_gain, float q_eps,
                                   float k_eps, const void* cos, const void* sin, int64_t table_rows,
                                   const int64_t* position, int positions, const int64_t* phases, void* keys,
                                   void* values, void* out, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                   int64_t capacity, int64_t dim, double scale, void* workspace,
                                   int64_t workspace_bytes, const ftk_attn_config* cfg, void* stream);
/* Workspace bytes of that call on the current device (-1: invalid shape or no device). */
int64_t ftk_decode_attention_workspace_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity,
                                             int64_t dim, const ftk_attn_config* cfg);
/* ---- Q/K head norm + RoPE + KV-cache update ---------------------------------------- */
#define FTK_ROPE_PREFILL 0x1  /* token t goes to cache slot t (else position + t) */
#define FTK_ROPE_ROWS 0x2     /* one position per batch row; cos/sin [B, T, D] (else [1, T, D] shared) */
#define FTK_ROPE_TABLE 0x4    /* cos/sin are whole [table_rows, D] tables; row b token t rotates at
                                 position[b] + phases[b, t] (needs FTK_ROPE_ROWS) */
/* For each row b (of `batch`), token t (of `tokens`) and head h of the packed QKV
 * [B, T, (Hq + 2 Hkv) D] (BF16, or `splits` > 1 FP32 partial planes `split_stride`
 * elements apart, summed and rounded to BF16): n = bf16(x / sqrt(mean(x^2) + eps)),
 * w = bf16(n * gain) with q_gain / q_eps for the Hq query heads and k_gain / k_eps
 * for the Hkv key heads, then out = bf16(bf16(w * cos) + bf16(rotate_half(w) * sin)).
 * Query heads go to query [B, T, Hq, D]; key heads to keys [B, Hkv, C, D] at the
 * step's slot, and the value heads are copied to values at the same slot. Slots
 * outside [0, capacity) and phases outside [0, table_rows) are skipped on the
 * device. D is 64 or 128; pointers 4-byte aligned. Replaces qk_rope_cache
 * (engine/kernels/qk_rope.py:13-129). */
int ftk_qk_rope_cache_bf16(const void* packed, int splits, int64_t split_stride, const void* q_gain,
                           const void* k_gain, float q_eps, float k_eps, const void* cos, const void* sin,
                           int64_t table_rows, const int64_t* position, const int64_t* phases, void* query,
                           void* keys, void* values, int64_t batch, int64_t tokens, int64_t q_heads,
                           int64_t kv_heads, int64_t capacity, int64_t dim, int mode, void* stream);
/* ---- measurement --------------------------------------------------------------- */
/* A pure streaming read of `bytes` (a multiple of 16, src 16-byte aligned) with the
 * projection kernels' load path: `grid` persistent workgroups of 256 lanes with a
 * rolling window of `loads` (2, 4, 8 or 16) 16-byte non-temporal loads per lane, or,
 * with grid 0, one-shot workgroups that each read 256 `loads` chunks (ceil(bytes /
 * (4096 loads)) of them) and exit; nothing computed but an XOR fold. sink: one
 * 32-bit word per workgroup, practically never written. Its time is the floor
 * a projection reading the same bytes in one launch is measured against (the
 * bandwidth reference of bench.py). No counterpart in the reference, which prices
 * its kernels against the nominal bandwidth only (agent/EXPERIMENTS.md:2231-2239). */
int ftk_stream_read(const void* src, int64_t bytes, void* sink, int grid, int loads, void* stream);

/* ---- planning (host only, no device needed) ---------------------------------- */
/* The launch ftk_decode_attention_bf16 would make on `compute_units` CUs. */
int ftk_plan_decode_attention(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity, int64_t dim,
                              int compute_units, const ftk_attn_config* cfg, ftk_attn_plan* plan);

/* The launch ftk_project_bf16 would make for this shape on `compute_units` CUs
 * (`epilogue` | FTK_PLAN_PROLOGUE for a call with gamma). */
int ftk_plan_project(int64_t M, int64_t N, int64_t K, int epilogue, int compute_units, const ftk_config* cfg,
                     ftk_plan* plan);

/* Replays `plan`'s tile walk on the host with the kernels' own index functions:
 * counts[c] = number of (workgroup, tile, wave, slot) writing output column c
 * (length outputs = N, or N/2 for SwiGLU); *max_row = largest weight row read. */
int ftk_plan_coverage(const ftk_plan* plan, int64_t N, int epilogue, int32_t* counts, int64_t outputs,
                      int64_t* max_row);

#ifdef __cplusplus
}
#endif

#endif /* FTK_H */
