/*
 * gatgpu.h -- C ABI of the MI355X (gfx950) three-layer multi-head GAT forward.
 *
 * One opaque context per device owns every device buffer: the destination-row
 * CSR graph, its degree schedule, three layers of weights and the per-layer
 * activations.  Host buffers stay owned by the caller.  No function throws;
 * each returns 0 (GATGPU_OK) or a negative error class, and
 * gatgpu_last_error() describes the failure.  A context is used by one host
 * thread at a time.
 *
 * The entry points replace the per-layer "paths" of the reference harness:
 *   run_path(path, g, p, q, s, input, w, hidden, panel, t, policy)
 *     baseline/bench/main.cpp:21-25 (path whitelist main.cpp:30)
 *   X_layer(const Graph&, const Param&, const Prepared&, [const Schedule&,]
 *           const std::vector<float>& input, Workspace&, bool hidden, Times&)
 *     baseline/include/gat.hpp:107-117
 * The graph container (u64 rowptr, u32 col, f32 x; baseline/include/gat.hpp:32-39)
 * and the weight layout (W[in][heads*dim] row-major, head h = columns
 * [h*dim,(h+1)*dim), aL/aR[heads*dim]; baseline/include/gat.hpp:42-48) are
 * taken unchanged.
 */
#ifndef GATGPU_H
#define GATGPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gatgpu_ctx gatgpu_ctx;

/* Return codes.  The reference throws std::runtime_error for each of these
 * (baseline/src/common.cpp:6-49); its harness maps them to "FAIL msg", exit 1
 * (baseline/bench/main.cpp:184). */
enum {
    GATGPU_OK = 0,
    GATGPU_EINVAL = -1,     /* malformed argument, CSR, shape or option       */
    GATGPU_ESTATE = -2,     /* call order: graph/layer/input not set yet      */
    GATGPU_ENODEV = -3,     /* no usable HIP device / wrong architecture      */
    GATGPU_ENOMEM = -4,     /* device allocation failed                       */
    GATGPU_EDEVICE = -5,    /* a HIP call or kernel launch failed             */
    GATGPU_ENONFINITE = -6, /* NaN/Inf in features or weights                 */
    GATGPU_EOVERFLOW = -7   /* size product overflows (common.cpp:6-9)        */
};

/* Precision of a forward.  FP32: FP32 X, W, Z and softmax state (the
 * reference's ref_fp32 / standard_fp32).  BF16: RNE-rounded bf16 X and W,
 * FP32 MFMA accumulation, L/R from the FP32 accumulators, Z stored bf16,
 * FP32 score/max/exp/denominator/output accumulation (standard_bf16 with a
 * bf16 copy of Z; baseline/IMPLEMENTATION_CONTRACT.md sections 3.2-3.3).
 * On transform-first layers of 8 heads x 32 features R is instead the FP32
 * dot of the stored bf16 Z row with a_r, formed both in the projection and,
 * per edge, in the aggregation from the Z row it gathers anyway, so no R
 * values are gathered; the row max stays exact over those R values. */
enum { GATGPU_FP32 = 0, GATGPU_BF16 = 1 };

/* Dataflow of one layer.  TRANSFORM_FIRST projects Z = X W then aggregates Z
 * rows (standard_layer, baseline/src/baseline_standard.cpp:98-108).
 * AGGREGATE_FIRST gathers the layer's input rows instead of Z
 * (tfs_online_fused, implementation/src/gat_tfs_online.cpp:200-283); bf16
 * only, in <= 128, and head_dim 32 with 1, 2, 4 or 8 heads or 8 heads of 64.
 * For 8 heads it runs in the sum form of tfs_online_fused: U_h = sum_j p_jh X_j
 * per row (FP32 sums of the bf16 rows, p entering as hi + lo bf16), then
 * (U_h / den_h) W_h on the MFMA units, with U_h / den_h entering as hi + lo
 * bf16 for FP32 outputs and as one bf16 for bf16-stored hidden outputs (the
 * rounding of a bf16 projection input); otherwise each gathered row is projected
 * and p (X_j W_h) summed, in the neighbour-step order of
 * baseline/src/baseline_tfs.cpp:16-110.  AUTO selects the sum form where it
 * applies (bf16) and the layer's bf16 Z table (n x heads x head_dim x 2 bytes)
 * exceeds 256 MB, and transform-first elsewhere.  gatgpu_model_forward with
 * AGGREGATE_FIRST uses it on the layers that support it and transform-first
 * on the others. */
/* TFS_B1 is the faithful neighbour-step TFS ("tfs_bf16",
 * baseline/src/baseline_tfs.cpp:16-110, max_prescan first): per step the
 * weighted source row p X_j is rounded to bf16 and multiplied by W_h with FP32
 * sums, the exact row max taken before any exponent.  Same shape limits as
 * AGGREGATE_FIRST; used for dataflow comparisons, not selected by AUTO. */
enum { GATGPU_AUTO = 0, GATGPU_TRANSFORM_FIRST = 1, GATGPU_AGGREGATE_FIRST = 2, GATGPU_TFS_B1 = 3 };

/* Stage selectors for gatgpu_get_stage (Workspace fields, gat.hpp:96-106). */
enum {
    GATGPU_STAGE_Z = 0,    /* [n][heads*dim] projected features (TF only)   */
    GATGPU_STAGE_LEFT = 1, /* [n][heads]                                     */
    GATGPU_STAGE_RIGHT = 2,/* [n][heads]                                     */
    GATGPU_STAGE_MAX = 3,  /* [n][heads] exact row max M = leaky(L + max R)  */
    GATGPU_STAGE_DEN = 4,  /* [n][heads] sum of exp(score - M)               */
    GATGPU_STAGE_OUT = 5,  /* [n][heads*dim] normalised (+ELU) layer output  */
    GATGPU_STAGE_XBF = 6   /* [n][in] the layer input rounded to bf16, as
                              convert() writes Workspace::xbf (common.cpp:
                              85-93): bf16 layers whose FP32 input the layer
                              rounds itself -- by the convert kernel, by the
                              projection (kept only with option
                              GATGPU_OPT_KEEP_INPUT_BF16) or into the
                              aggregate-first gather table.  Absent for a
                              chained bf16 input: that is the previous
                              layer's OUT stage, rounded in its epilogue.  */
};

/* Per-layer stage times in milliseconds, measured with HIP events on the
 * context's stream.  Field names follow gat::Times (baseline/include/gat.hpp:68-76).
 * normalize and activation are fused into the aggregation kernel on the GPU,
 * so their time is inside aggregate_ms and their fields read 0. */
typedef struct gatgpu_times {
    double convert_ms;
    double projection_ms;
    double lr_ms;
    double max_prescan_ms;
    double aggregate_ms;
    double normalize_ms;
    double activation_ms;
    double total_ms;
} gatgpu_times;

/* Options (gatgpu_set_option).  Thresholds are in-degrees. */
enum {
    GATGPU_OPT_BLOCK_ROW_MIN_DEGREE = 1, /* rows at/above use a block per row  */
    GATGPU_OPT_SPLIT_ROW_MIN_DEGREE = 2, /* rows at/above are split over waves
                                            (default per kernel: 1024 sum form,
                                            1536 8-head, 2048 one-head; 512 on
                                            graphs below 16M edges; chunks
                                            doubled until the heaviest row has
                                            <= 96 of them, the degree with them
                                            (8-head) or at least 2 chunks (the
                                            others); a value applies to all,
                                            0 restores them)                  */
    GATGPU_OPT_SPLIT_CHUNK_EDGES = 3,    /* edges per split chunk (default per
                                            kernel: 256, 512, 1024; 256 below
                                            16M edges; scaled as above; a value
                                            >= 64 applies to all, 0 restores) */
    /* 4 is not a key: rows of small degree take one wave each like the rest
       (the one-head kernel already packs 8 rows of equal degree per wave). */
    GATGPU_OPT_KEEP_INPUT_BF16 = 5,      /* 1: bf16 transform-first layers also
                                            store the input rows their
                                            projection rounds (stage XBF);
                                            0 (default): they are rounded in
                                            registers only                    */
    GATGPU_OPT_FUSE_NEXT_PROJECTION = 6  /* 2: gatgpu_model_forward runs the
                                            projection of a bf16 one-head
                                            output layer (<= 60 classes over
                                            8 x 32 inputs) inside the previous
                                            layer's aggregation, on its output
                                            rows staged in LDS: Z, L and R of
                                            the output layer are bit-equal to
                                            the unfused run, and the hidden
                                            layer's OUT stage is not stored
                                            (gatgpu_stage_size gives 0, and a
                                            per-layer forward of the output
                                            layer chained on it fails).
                                            1 (default): the same on graphs of
                                            at least 16M edges, where it is the
                                            faster form; smaller graphs run
                                            unfused.
                                            0: every layer stores its output  */
};

/* ---- lifetime -------------------------------------------------------- */
/* Opens `device` (HIP ordinal), checks it is a gfx950, creates the stream. */
int gatgpu_create(int device, gatgpu_ctx** out);
/* Frees every device buffer; accepts NULL. */
int gatgpu_destroy(gatgpu_ctx* ctx);
/* Message of the last failure on ctx (or of the last failed create when ctx
 * is NULL).  Valid until the next call on the same context. */
const char* gatgpu_last_error(const gatgpu_ctx* ctx);

/* ---- static inputs (untimed, like load_graph/prepare: baseline/README.md:52) ---- */
/* The host checks of gatgpu_set_graph without a context or device
 * (Graph::validate, baseline/src/common.cpp:23-30): row[0] == 0, row[n] == e,
 * monotone rows, col[k] < n, 0 < n <= INT32_MAX, e <= 2^40, and every
 * in-degree below 2^32 (GATGPU_EOVERFLOW).  Rows are checked before sources.
 * The message is gatgpu_last_error(NULL). */
int gatgpu_validate_graph(uint64_t n, uint64_t e, const uint64_t* row, const uint32_t* col);
/* Validates (as gatgpu_validate_graph) and uploads the CSR, then builds the
 * degree schedule on the GPU.  Replaces load_graph + Graph::validate
 * (baseline/src/common.cpp:23-39) and degree_schedule (common.cpp:120-125). */
int gatgpu_set_graph(gatgpu_ctx* ctx, uint64_t n, uint64_t e, const uint64_t* row,
                     const uint32_t* col);
/* Uploads one layer (0..2) of weights and prepares its bf16 copy.  Replaces
 * Param::validate + prepare (common.cpp:45-49, 97-119): 0 < heads <= 8,
 * 0 < dim <= 64, 0 < in, all values finite. */
int gatgpu_set_layer(gatgpu_ctx* ctx, int layer, int in, int heads, int dim, const float* w,
                     const float* al, const float* ar);
/* Uploads the node features x[n][din] (Graph::x); all values finite. */
int gatgpu_set_input(gatgpu_ctx* ctx, uint64_t n, int din, const float* x);

/* ---- schedule -------------------------------------------------------- */
/* Copies the degree permutation (perm[sorted] = original row, ascending
 * (degree, id)) and neighbor_steps (sum over 16-row tiles of the last row's
 * degree), both computed on the GPU.  Either pointer may be NULL.
 * Replaces degree_schedule (baseline/src/common.cpp:120-125) and degree_perm
 * (implementation/src/gat_tfs_online.cpp:180-189). */
int gatgpu_degree_schedule(gatgpu_ctx* ctx, uint32_t* perm, uint64_t* neighbor_steps);
/* Copies the CSR in degree-sorted order: prow[k] = sum of degrees of
 * perm[0..k), pcol[prow[k]..prow[k+1]) = col[row[perm[k]]..row[perm[k]+1]). */
int gatgpu_permuted_csr(gatgpu_ctx* ctx, uint64_t* prow, uint32_t* pcol);
/* choose_R (implementation/src/gat_tfs_online.cpp:191-199) from the device
 * max degree: 128 if rho<32, 64 if rho<1024, 32 if rho<20000, else 16. */
int gatgpu_choose_R(gatgpu_ctx* ctx, int* r_out);

/* ---- forward --------------------------------------------------------- */
/* One layer (0..2).  `input` NULL chains from the device-resident output of
 * layer-1 run with the same precision (layer 0 reads the graph features);
 * non-NULL uploads a host FP32 [n][in] matrix first (outside the timing),
 * as run_path takes any `input` vector.  hidden != 0 applies ELU
 * (layers 0 and 1 of the model).  times may be NULL.
 * Replaces standard_layer / ref_layer / tfs_layer (gat.hpp:107-117) and
 * reference / tfs_online_fused (implementation/src/gat_online.cpp:167,
 * implementation/src/gat_tfs_online.cpp:200-202). */
int gatgpu_layer_forward(gatgpu_ctx* ctx, int layer, int precision, int dataflow, int hidden,
                         const float* input, gatgpu_times* times);
/* The three layers chained on device (hidden = layer < 2), timed from the
 * first kernel of layer 0 to the last of layer 2 with HIP events (the model
 * timer of baseline/bench/main.cpp:171-174).  logits (NULL allowed) receives
 * layer 2's FP32 [n][dim] output after the timer stops.  times (NULL allowed)
 * points at 3 per-layer records; total_ms (NULL allowed) gets the model time.
 * The per-stage events are recorded only when times is given: with total_ms
 * alone the forward carries two events, its first and its last.
 * dataflow applies to every layer (AUTO decides per layer; AGGREGATE_FIRST
 * falls back to transform-first on layers it does not support). */
int gatgpu_model_forward(gatgpu_ctx* ctx, int precision, int dataflow, float* logits,
                         gatgpu_times* times, double* total_ms);
/* ---- fixed-p operator ----------------------------------------------- */
/* Uploads a fixture's attention weights for `layer`: p[e][heads] (the
 * unnormalised exp weights, original CSR edge order) and den[n][heads].
 * Checks them as load_fixture does (baseline/src/common.cpp:186-193): all
 * finite, p in [0, 1], den equal to the row's sum of p within 1e-5 relative,
 * den > 0 on a non-empty row.  p is permuted to degree-sorted order on the
 * device.  set_graph and set_layer(layer) drop the fixture.  The GATFIX1 file
 * (common.cpp:171-194) is read by the host harness. */
int gatgpu_set_fixed_p(gatgpu_ctx* ctx, int layer, const float* p, const float* den);
/* The fixed-p operator of the reference harness (baseline/bench/main.cpp:
 * 103-150, "standard_op"): projection Z = XW in `precision`, then
 * out = (sum_e p[e] Z[col[e]]) * (den > 0 ? 1/den : 0) with the fixture's p
 * and den and no activation (standard_aggregate with fixed_p and finish,
 * baseline/src/baseline_standard.cpp:52-97).  dataflow TFS_B1 is the
 * reference's "tfs_op" of the same mode (tfs_aggregate with fixed_p,
 * baseline_tfs.cpp:16-110), AGGREGATE_FIRST the FP32-product variant; both
 * bf16 only.  input as in gatgpu_layer_forward.  Stages: Z (transform-first),
 * LEFT, RIGHT from the projection, DEN = the fixture's den, MAX zero, OUT FP32. */
int gatgpu_fixed_p_forward(gatgpu_ctx* ctx, int layer, int precision, int dataflow, const float* input,
                           gatgpu_times* times);

/* Copies a stage of the last forward of `layer` as FP32 (bf16 stages are
 * widened exactly). */
int gatgpu_get_stage(gatgpu_ctx* ctx, int layer, int which, float* host_out);
/* Size in floats of a stage buffer (0 if absent). */
int gatgpu_stage_size(gatgpu_ctx* ctx, int layer, int which, uint64_t* count);

/* Wall-clock times (ms) of the static steps, outside every forward timer
 * (the reference prints them as STATIC degree_sort_ms / model_prepare_ms and
 * COLD startup_before_inference_ms, baseline/bench/main.cpp:56,168-169;
 * baseline/README.md:52).  Each field holds its step's last run. */
typedef struct gatgpu_static_times {
    double graph_check_ms;   /* set_graph: host CSR validation (Graph::validate)      */
    double graph_h2d_ms;     /* set_graph: rowptr and col upload                     */
    double degree_sort_ms;   /* set_graph: degree schedule on the device (sort,
                                permuted CSR, relabelling, split tables)             */
    double model_prepare_ms; /* set_layer: checks, bf16 W, B_LR, fragment packing
                                and upload, summed over the layers set             */
    double input_h2d_ms;     /* set_input: feature checks and upload                 */
    double input_permute_ms; /* set_input: features gathered into degree order       */
    double logits_d2h_ms;    /* model_forward: the logits copied to the host         */
} gatgpu_static_times;
int gatgpu_get_static_times(gatgpu_ctx* ctx, gatgpu_static_times* out);

/* ---- allocation-free layer ------------------------------------------- */
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops): the
 * transform-first gatgpu_layer_forward of `layer` on device-resident rows,
 * with every intermediate (bf16 input rows, Z, L, R, max, den, the output
 * before its final copy, split-row partial sums and arrival counters) in one
 * static device array of GATGPU_STATIC_SCRATCH_BYTES per GPU, held until the
 * process ends.  It calls no allocator.
 *   x   device FP32 [n][in], original node order
 *   out device FP32 [n][heads*dim], original node order: the values
 *       gatgpu_get_stage(OUT) returns after gatgpu_layer_forward with the
 *       same input, precision and hidden (bf16 hidden outputs widened)
 * Graph, layer weights and options come from the context (set-up calls,
 * which do allocate).  The work is enqueued on the context's stream
 * (gatgpu_stream) and the call returns without waiting; the stages of the
 * context are not touched.  Rejects (GATGPU_EOVERFLOW, before any launch) a
 * layer whose intermediates exceed the array.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (several contexts or host
 * threads, or streams not ordered against each other) race. */
#define GATGPU_STATIC_SCRATCH_BYTES (64u << 20)
int gatgpu_layer_forward_static(gatgpu_ctx* ctx, int layer, int precision, int hidden, const float* x,
                                float* out);
/* Bytes of the static array gatgpu_layer_forward_static would use for
 * `layer` of the context's graph.  GATGPU_ESTATE (and *bytes untouched) if
 * the graph or the layer's weights are not set. */
int gatgpu_static_scratch_need(gatgpu_ctx* ctx, int layer, int precision, int hidden, uint64_t* bytes);

/* ---- misc ------------------------------------------------------------ */
int gatgpu_set_option(gatgpu_ctx* ctx, int key, int64_t value);
/* Blocks until all work on the context's stream is done. */
int gatgpu_synchronize(gatgpu_ctx* ctx);
/* The context's HIP stream (hipStream_t) for callers that order their own
 * work against it. */
void* gatgpu_stream(gatgpu_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif /* GATGPU_H */
