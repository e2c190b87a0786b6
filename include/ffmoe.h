/*
 * ffmoe.h -- C ABI of libffmoe.so, the MI355X (gfx950) kernels of the fused
 * Mixture-of-Experts layer (non-expert-parallel path).
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are DEVICE pointers owned by the caller (the torch
 *     caching allocator); the library never allocates device memory.
 *   - Tensors are dense and row-major.  "bf16" is IEEE bfloat16 stored as
 *     uint16_t; int64 index tensors match torch.int64.
 *   - `stream` is a hipStream_t passed as void*; every kernel is enqueued on it
 *     and nothing synchronises the host.
 *   - Return value: 0 on success.  Nonzero means the arguments were rejected
 *     (nothing was launched) or a launch failed; ffmoe_last_error() returns a
 *     message describing the most recent failure on the calling thread.
 *
 * Token/row vocabulary (identical to the reference's)
 *   N tokens, D model dim, E experts, k = top_k, H = ffn_dim / 2.
 *   Entry j = n*k + s is token n's s-th choice (slot).  Each expert's entries
 *   are ranked in ascending j (the reference's stable argsort,
 *   fused_moe.py:344-348).  Entries of expert e with rank < mt own a row of the
 *   expert-sorted activation matrix; this library stores those rows COMPACTLY:
 *   row = offsets[e] + rank, offsets[e] = sum_{e'<e} min(count[e'], mt).  The
 *   reference's padded coordinate is e*mt + rank (moe_ops.py:84-98); both name
 *   the same permutation.  row_of[j] holds the row, or
 *     FFMOE_ROW_DROPPED (-1): entry dropped, contributes zero (capacity
 *                              sentinel row, fused_moe.py:428-430), or
 *     FFMOE_ROW_ALIAS0  (-2): entry overflowed mt and reads row 0 like the
 *                              reference's e2b = 0 (moe_ops.py:87-91, :138-140).
 */
#ifndef FFMOE_H
#define FFMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FFMOE_ROW_DROPPED (-1)
#define FFMOE_ROW_ALIAS0 (-2)

/* gating */
#define FFMOE_GATING_SOFTMAX 0
#define FFMOE_GATING_SIGMOID 1
/* activation */
#define FFMOE_ACT_SWIGLU 0
#define FFMOE_ACT_GEGLU 1 /* tanh-approximated GELU (the routed experts, activations.py) */
#define FFMOE_ACT_RELU2 2
#define FFMOE_ACT_GEGLU_ERF 3 /* exact erf GELU (the shared expert's F.gelu, nn.py:36) */

/* compute dtype of the ffmoe_t_* entry points (the fp32 / fp64 path) */
#define FFMOE_DTYPE_F32 1
#define FFMOE_DTYPE_F64 2

/* limits enforced by the entry points */
#define FFMOE_MAX_EXPERTS 256
#define FFMOE_MAX_TOPK 16
/* Largest expert count for which the gate-gradient products run in the
 * fused kernels below (ffmoe_dx_reduce, ffmoe_gate_grad). */
#define FFMOE_MAX_FUSED_GATE_E 32

/* layout of the `stats` output of ffmoe_route_scan (fp32 slots) */
#define FFMOE_STAT_AUX 0          /* aux_loss (coefficient applied)            */
#define FFMOE_STAT_Z 1            /* z_loss (coefficient applied)              */
#define FFMOE_STAT_IMBALANCE 2    /* max count / (mean count + 1e-6)           */
#define FFMOE_STAT_DROP_FRAC 3    /* dropped entries / (N*k)                   */
#define FFMOE_NUM_STATS 4
/* layout of the `istats` output of ffmoe_route_scan (int32 slots) */
#define FFMOE_ISTAT_MAX 0         /* max tokens_per_expert                     */
#define FFMOE_ISTAT_MIN 1         /* min tokens_per_expert                     */
#define FFMOE_ISTAT_DROPPED 2     /* entries without a row (rank >= mt)        */
#define FFMOE_NUM_ISTATS 4

/* Message for the most recent failure on this thread ("" if none). */
const char* ffmoe_last_error(void);

/* Library version, for the loader's sanity check. */
int ffmoe_version(void);

/* ------------------------------------------------------------------------ */
/* Routing forward                                                          */
/* ------------------------------------------------------------------------ */

/* Bytes of workspace ffmoe_route_fwd / ffmoe_route_scan / ffmoe_permute share
 * for a problem of N tokens, E experts and top_k = k.  The same workspace
 * (and the same N, E, k) must be passed to all three calls of one forward. */
size_t ffmoe_route_workspace_bytes(int64_t N, int E, int k);

/* Gate GEMM + scoring + top-k + per-block routing statistics.
 * Replaces: the gate GEMM `hidden @ gate.T` (fused_moe.py:334, :1165),
 *   `fused_topk_routing` and its kernels (fused_topk.py:30-179, via
 *   `_apply_routing` fast path fused_moe.py:139-142), the `bincount` and
 *   per-expert sums of the losses block (fused_moe.py:1176-1194).
 * x [N,D] bf16, gate [E,D] bf16.  If logits_in != NULL the gate GEMM is
 * skipped and those bf16 logits [N,E] are routed instead (the reference's
 * `fused_topk_routing(logits, ...)` boundary); otherwise the bf16 logits are
 * written to logits_out [N,E] (may be NULL).
 * expert_bias [E] fp32 or NULL: added to the scores for SELECTION only
 *   (fused_moe.py:163-179, :183-193); weights use unbiased scores.
 * Outputs: topk_idx [N,k] int64, topk_w [N,k] fp32 (slots in descending
 *   selection order; lowest expert index wins a tie, fused_topk.py:63-70),
 *   lse [N] fp32 (logsumexp of the fp32 logits; may be NULL).
 * Selection rule, weights: softmax over the selected logits, or sigmoid
 *   scores / (sum + 1e-6) (fused_topk.py:72-78, :128-132).
 * need_sigmoid_sum: also accumulate sum_n sigmoid(logit) per expert (the
 *   sigmoid aux loss, fused_moe.py:1187-1188). */
int ffmoe_route_fwd(const void* x, const void* gate, const void* logits_in,
                    const float* expert_bias, int64_t N, int D, int E, int k,
                    int gating, int need_sigmoid_sum, void* logits_out,
                    int64_t* topk_idx, float* topk_w, float* lse,
                    void* workspace, void* stream);

/* ffmoe_route_fwd with the routing options of the reference's slow path
 * (`_apply_routing`, fused_moe.py:116-200, and `_group_limited_topk`
 * :203-251, with the input jitter of :329-332):
 *   expert_bias      [E] fp32, added to the selection scores only;
 *   bias_round_bf16  1 when the caller's bias is bf16 (softmax gating without
 *                    pre_softmax adds it to the bf16 logits in bf16);
 *   pre_softmax      softmax over all experts before selection, weights the
 *                    selected probabilities renormalised (+1e-6);
 *   scoring_factor   > 0: weights scaled by scoring_factor / k;
 *   n_group, topk_group  > 0: group-limited selection (E % n_group == 0);
 *   jitter_noise     [N,D] bf16 or NULL: logits from bf16(x * noise).
 * Selection ties go to the lower index (groups and experts). */
int ffmoe_route_fwd_ex(const void* x, const void* gate, const void* logits_in,
                       const float* expert_bias, int bias_round_bf16,
                       int pre_softmax, float scoring_factor, int n_group,
                       int topk_group, const void* jitter_noise, int64_t N, int D,
                       int E, int k, int gating, int need_sigmoid_sum,
                       void* logits_out, int64_t* topk_idx, float* topk_w,
                       float* lse, void* workspace, void* stream);

/* Global prefix over the per-block expert histograms, losses and metrics.
 * Replaces: `bincount`/`cumsum` (fused_moe.py:346-348), the overflow check's
 *   max (fused_moe.py:401), the aux/z-loss and metrics reductions
 *   (fused_moe.py:1176-1217).
 * mt: rows per expert (max_tokens, or the capacity when capacity dropping).
 * gemm_bm: row-tile height of the grouped GEMMs; tile_offsets[e] is the
 *   number of gemm_bm-row tiles of experts < e.
 * Outputs: counts [E] int32 (tokens_per_expert), offsets [E+1] int32,
 *   tile_offsets [E+1] int32, stats [FFMOE_NUM_STATS] fp32,
 *   istats [FFMOE_NUM_ISTATS] int32.  * aux_out / z_out (may be NULL): single-float copies of stats[AUX] and
 *   stats[Z], so a caller can hand the losses out as separate tensors. */
int ffmoe_route_scan(int64_t N, int E, int k, int mt, int gemm_bm,
                     float aux_coeff, float z_coeff, int gating,
                     void* workspace, int32_t* counts, int32_t* offsets,
                     int32_t* tile_offsets, float* stats, int32_t* istats,
                     float* aux_out, float* z_out, void* stream);

/* Stable permutation of tokens into expert-sorted compact rows.
 * Replaces: `fused_routing_scatter` (moe_ops.py:43-149) and the capacity
 *   keep-mask / renormalisation (fused_moe.py:350-390, :428-430).
 * x [N,D] bf16 -> x_sorted [rows, D] bf16 (rows = offsets[E]), row_of [N*k].
 * capacity_mode: 1 = entries with rank >= mt are dropped (FFMOE_ROW_DROPPED)
 *   and topk_w is renormalised in place; 0 = overflow entries alias row 0
 *   (FFMOE_ROW_ALIAS0) when expert 0 has a row, else FFMOE_ROW_DROPPED. */
int ffmoe_permute(const void* x, const int64_t* topk_idx, float* topk_w,
                  const int32_t* offsets, const int32_t* counts, int64_t N, int D,
                  int E, int k, int mt, int capacity_mode, void* workspace,
                  void* x_sorted, int32_t* row_of, void* stream);

/* ------------------------------------------------------------------------ */
/* Expert grouped GEMMs (bf16 MFMA, fp32 accumulate, bf16 out).             */
/* Row groups come from offsets[E+1] and tile_offsets[E+1] on the device;   */
/* tile_offsets must have been computed (ffmoe_route_scan's gemm_bm) for    */
/* the same tile_rows; max_rows is the host-side upper bound of offsets[E]  */
/* (N*k).                                                                   */
/* ------------------------------------------------------------------------ */

/* Row-tile height the grouped GEMMs use for max_rows rows over E experts
 * (128 or 256).  Pass it as `gemm_bm` to ffmoe_route_scan and as `tile_rows`
 * to the grouped GEMMs.  No reference counterpart (the reference pads every
 * expert to max_tokens rows). */
int ffmoe_gemm_tile_rows(int64_t max_rows, int E);

/* Bytes of the `sk_workspace` the four grouped-rows GEMMs below take on the
 * current device (-1 if the device cannot be queried).  Its first 8 KiB and
 * its last 64 KiB are int32 flags that must be zero before the first call
 * (allocate it zeroed); every call leaves them zero again, so one workspace
 * serves any number of calls in stream order.
 * Calls that may overlap (different streams) need separate workspaces.
 * With sk_workspace NULL the GEMMs run one block per tile instead of the
 * persistent one-block-per-CU schedule whose last round is split along K.
 * No reference counterpart (the reference's GEMMs are cuBLAS bmm calls). */
int64_t ffmoe_gemm_workspace_bytes(void);

/* A dense row group computed in the same launch as the routed experts (the
 * shared expert of MoELayer, nn.py:22-44, :156-159): its row tiles follow
 * the routed tiles of each *_shared GEMM below, with the same K and N as one
 * routed expert.  For the grouped-rows GEMMs `a` holds its A rows
 * [rows, K], `b` its weight matrix (laid out as one routed expert's), `c`
 * its output rows, `c2` (GLU forward, may be NULL) its pre-activation
 * output, `up` (GLU backward) its pre-activation input; for
 * ffmoe_gemm_wgrad_shared it is group E, K = its rows: c [M, Nc] =
 * a[rows, M]^T · b[rows, Nc].  `activation` is its GLU (FFMOE_ACT_*). */
typedef struct ffmoe_dense_group {
  const void* a;
  const void* b;
  const void* up;
  void* c;
  void* c2;
  int64_t rows;
  int activation;
} ffmoe_dense_group;

/* The grouped-rows GEMMs with a dense extra group in the same launch
 * (shared may be NULL: then identical to the plain entry points).  No
 * reference counterpart (the reference runs the shared expert as three
 * nn.Linear modules outside the fused op). */
int ffmoe_gemm_up_glu_shared(const void* x_sorted, const void* w_up, const int32_t* offsets,
                             const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                             int D, int H, int activation, void* up_out, void* act_out,
                             const ffmoe_dense_group* shared, void* sk_workspace, void* stream);
int ffmoe_gemm_down_shared(const void* act, const void* w_down, const int32_t* offsets,
                           const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                           int H, int D, void* down_out, const ffmoe_dense_group* shared,
                           void* sk_workspace, void* stream);
/* ffmoe_gemm_up_glu_shared followed by ffmoe_gemm_down_shared on its
 * act_out (shared_down->a must be shared_up->c), as one persistent launch
 * where it applies (tile_rows 256, D and H multiples of 64, D below 4096,
 * sk_workspace given): a row tile's down tiles start as soon as all its up
 * tiles are done, so they fill the up GEMM's last, partial round.  The
 * outputs are those of the two calls (bit for bit those of the two calls
 * with sk_workspace NULL: no tile's K range is split), which it makes
 * itself where the fused schedule does not apply.  Replaces: the up bmm + activation and the
 * down bmm (fused_moe.py:435-441). */
int ffmoe_gemm_up_down_shared(const void* x_sorted, const void* w_up, const void* w_down,
                              const int32_t* offsets, const int32_t* tile_offsets, int tile_rows,
                              int E, int64_t max_rows, int D, int H, int activation, void* up_out,
                              void* act_out, void* down_out, const ffmoe_dense_group* shared_up,
                              const ffmoe_dense_group* shared_down, void* sk_workspace, void* stream);
/* ffmoe_gemm_wgrad_shared(gup, x_sorted, offsets, E, 2H, D, dwu_out,
 * shared_wgrad, ...) and ffmoe_gemm_dgrad_shared(gup, w_up, ..., ghb_out,
 * shared_dgrad, ...) as one persistent launch where it applies (a
 * workspace, 2H a multiple of 64, tile_rows 128 or 256): the two read the
 * same gup and are independent, so their tiles run as one list, dgrad's
 * first, with no stream-K partials.  The outputs are those of the two
 * calls (bit for bit those with sk_workspace NULL, where no tile's K range
 * is split), which it makes itself where the fused schedule does not
 * apply.  Replaces: the dX bmm of the up projection and its weight-gradient
 * bmm (fused_moe.py:553, :565). */
int ffmoe_gemm_dgrad_wgrad_shared(const void* gup, const void* w_up, const void* x_sorted,
                                  const int32_t* offsets, const int32_t* tile_offsets, int tile_rows,
                                  int E, int64_t max_rows, int H, int D, void* ghb_out, void* dwu_out,
                                  const ffmoe_dense_group* shared_dgrad,
                                  const ffmoe_dense_group* shared_wgrad, void* sk_workspace, void* stream);
int ffmoe_gemm_dgrad_glu_shared(const void* wgo, const void* w_down, const void* up,
                                const int32_t* offsets, const int32_t* tile_offsets,
                                int tile_rows, int E, int64_t max_rows, int D, int H,
                                int activation, void* gup_out, const ffmoe_dense_group* shared,
                                void* sk_workspace, void* stream);
int ffmoe_gemm_dgrad_shared(const void* gup, const void* w_up, const int32_t* offsets,
                            const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                            int H, int D, void* ghb_out, const ffmoe_dense_group* shared,
                            void* sk_workspace, void* stream);
/* ffmoe_gemm_wgrad_shared: with sk_workspace (the persistent GEMMs'
 * workspace, ffmoe_gemm_workspace_bytes) and a dense group of at least 4096
 * rows, the group's K is cut into two halves finished through the
 * workspace (the sum of the two fp32 halves: the same bits whichever half
 * finishes first); NULL keeps one K range per tile. */
int ffmoe_gemm_wgrad_shared(const void* a, const void* b, const int32_t* offsets, int E, int M,
                            int Nc, void* c_out, const ffmoe_dense_group* shared,
                            void* sk_workspace, void* stream);

/* Reports a failed stream-K partner wait of an earlier grouped GEMM on
 * sk_workspace.  The wait is bounded; it is not expected to time out (the
 * block it waits for is already running), but if it does the GEMM's output
 * is wrong and the kernel sets an error word in the workspace.  This call
 * synchronises `stream`, reads that word and returns 0 if it is clear;
 * otherwise it zeroes the workspace's flags (so later calls are sound again)
 * and returns nonzero with the message in ffmoe_last_error().  No reference
 * counterpart (the reference's GEMMs are cuBLAS bmm calls, which report no
 * such condition). */
int ffmoe_gemm_check(void* sk_workspace, void* stream);

/* up = x_sorted · w_up[e]^T and the fused GLU:
 *   up_out [rows, 2H] (pre-activation, may be NULL), act_out [rows, H].
 * Replaces: up bmm (fused_moe.py:435) + `activation_forward`
 *   (activations.py:27-74, :145-186).  w_up [E, 2H, D]: rows [0,H) gate half,
 *   [H,2H) up half. */
int ffmoe_gemm_up_glu(const void* x_sorted, const void* w_up,
                      const int32_t* offsets, const int32_t* tile_offsets,
                      int tile_rows, int E, int64_t max_rows, int D, int H,
                      int activation, void* up_out, void* act_out, void* sk_workspace,
                      void* stream);

/* down [rows, D] = act · w_down[e]^T.  w_down [E, D, H].
 * Replaces: down bmm (fused_moe.py:441). */
int ffmoe_gemm_down(const void* act, const void* w_down, const int32_t* offsets,
                    const int32_t* tile_offsets, int tile_rows, int E,
                    int64_t max_rows, int H, int D, void* down_out, void* sk_workspace,
                    void* stream);

/* gup [rows, 2H] = GLU_backward(wgo · w_down[e], up).
 * Replaces: dX-down bmm (fused_moe.py:547) + `activation_backward`
 *   (activations.py:77-142, :189-231). */
int ffmoe_gemm_dgrad_glu(const void* wgo, const void* w_down, const void* up,
                         const int32_t* offsets, const int32_t* tile_offsets,
                         int tile_rows, int E, int64_t max_rows, int D, int H,
                         int activation, void* gup_out, void* sk_workspace, void* stream);

/* ghb [rows, D] = gup · w_up[e].  Replaces: dX-up bmm (fused_moe.py:553). */
int ffmoe_gemm_dgrad(const void* gup, const void* w_up, const int32_t* offsets,
                     const int32_t* tile_offsets, int tile_rows, int E,
                     int64_t max_rows, int H, int D, void* ghb_out, void* sk_workspace,
                     void* stream);

/* Selects how MN-contiguous GEMM operands are read from LDS: 1 (default) =
 * ds_read_b64_tr_b16 transpose reads, 0 = element-wise reads.  Returns the
 * previous setting.  Both give identical results; the switch exists so the
 * transpose-read path can be verified against the element-wise one.  No
 * reference counterpart. */
int ffmoe_set_lds_transpose(int enable);

/* c[e] [M, Nc] = a[rows_e]^T · b[rows_e]; a [rows, M], b [rows, Nc].
 * Experts with no rows get zeros.
 * Replaces: dW-down and dW-up bmm (fused_moe.py:564-565). */
int ffmoe_gemm_wgrad(const void* a, const void* b, const int32_t* offsets, int E,
                     int M, int Nc, void* c_out, void* stream);

/* ------------------------------------------------------------------------ */
/* Combine / routing backward / dX reduce                                   */
/* ------------------------------------------------------------------------ */

/* out[n] = sum_s w[n,s] * rows[row_of[n*k+s]] accumulated in fp32 in slot
 * order; w is bf16(topk_w) (fused_moe.py:412) or, if topk_w is NULL, 1.
 * addend [N,D] bf16 or NULL: out = bf16(bf16(sum) + addend) (the reference's
 * `grad_hidden + gl @ gate`, fused_moe.py:590).
 * Replaces: `fused_gather_reduce` (moe_ops.py:156-241). */
int ffmoe_combine(const void* rows, const int32_t* row_of, const float* topk_w,
                  const void* addend, int64_t N, int D, int k, void* out,
                  void* stream);

/* dX reduce with the gate term: out[n] = bf16(bf16(sum_s ghb[row_of[n*k+s]])
 *   + bf16(gl[n,:] . gate)), slot sum fp32 in slot order, gl . gate fp32 over
 *   experts in index order.  gl [N,E] bf16, gate [E,D] bf16, E <=
 *   FFMOE_MAX_FUSED_GATE_E.
 * Replaces: the dX gather-reduce (fused_moe.py:556-561) and `gl @ gate`
 *   added to it (fused_moe.py:590). */
int ffmoe_dx_reduce(const void* ghb, const int32_t* row_of, const void* gl,
                    const void* gate, int64_t N, int D, int E, int k, void* out,
                    void* stream);

/* Bytes of fp32 partials ffmoe_gate_grad needs for N tokens. */
int64_t ffmoe_gate_grad_workspace_bytes(int64_t N, int D, int E);

/* dgate [E,D] bf16 = gl^T · x, fp32 accumulation in a fixed order.  Up to
 * FFMOE_MAX_FUSED_GATE_E experts a token-chunked bf16 dot2 kernel; above
 * that (E a multiple of 8, at most 256) the MFMA GEMM pipeline with the
 * token dimension split across blocks and the fp32 partials reduced in
 * split order.  Replaces: `gl.t() @ hidden` (fused_moe.py:591). */
int ffmoe_gate_grad(const void* gl, const void* x, int64_t N, int D, int E,
                    void* workspace, void* dgate, void* stream);

/* Bytes of fp32 partials ffmoe_gate_logits needs (0 when it does not split
 * the reduction). */
int64_t ffmoe_gate_logits_workspace_bytes(int64_t N, int D, int E);

/* logits [N,E] bf16 = x [N,D] · gate [E,D]^T on the MFMA GEMM pipeline (fp32
 * accumulation; the D reduction split across blocks when the tiles alone do
 * not fill the GPU, fp32 partials reduced in split order, one bf16 rounding).
 * D a multiple of 64, E a multiple of 8 (at most 256).  For gate matrices
 * too large for the route kernel's own gate GEMM, whose logits are then
 * passed to ffmoe_route_fwd as logits_in.
 * Replaces: the gate GEMM `hidden @ gate.T` (fused_moe.py:334, :1165). */
int ffmoe_gate_logits(const void* x, const void* gate, int64_t N, int D, int E,
                      void* logits, void* workspace, void* stream);

/* out [N,D] bf16 = gl [N,E] · gate [E,D] on the MFMA GEMM pipeline (fp32
 * accumulation, one bf16 rounding); E a multiple of 64 (at most 256), D a
 * multiple of 8.  The addend of ffmoe_combine for the dX reduce above
 * FFMOE_MAX_FUSED_GATE_E experts.  Replaces: `gl @ gate` (fused_moe.py:590). */
int ffmoe_gate_dx(const void* gl, const void* gate, int64_t N, int D, int E,
                  void* out, void* stream);

/* ffmoe_gate_grad without a workspace argument and without any allocation:
 * the fp32 partials live in a device array of
 * ffmoe_gate_grad_noalloc_max_bytes() bytes (32 MiB) that the library holds
 * on each device until the process ends.  Problems whose partials need more
 * (ffmoe_gate_grad_workspace_bytes(N, D, E) > that) are rejected.  Every
 * call on a device shares that device's array: calls that overlap on one
 * GPU (different streams or threads) race.  No counterpart in the reference;
 * it exists for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int64_t ffmoe_gate_grad_noalloc_max_bytes(void);
int ffmoe_gate_grad_noalloc(const void* gl, const void* x, int64_t N, int D, int E,
                            void* dgate, void* stream);

/* Routing backward, one pass per token.
 * Replaces: routing-weight grad (fused_moe.py:527-535), `fused_weighted_scatter`
 *   (moe_ops.py:248-332), softmax/sigmoid top-k backward + scatter_add
 *   (fused_moe.py:567-589), and the z-loss / sigmoid aux-loss gradients that
 *   autograd produces through the losses block (fused_moe.py:1178-1194).
 * go [N,D] bf16, down [rows,D] bf16, row_of [N*k], topk_idx, topk_w fp32,
 * logits [N,E] bf16, lse [N] fp32, counts [E] int32.
 * g_aux, g_z: fp32 device scalars (upstream grads of the losses) or NULL.
 * capacity_mode: 1 -> grads of tokens whose kept weights sum to 0 are zeroed
 *   (fused_moe.py:569-571).
 * Outputs: wgo [rows, D] bf16 (go[n] * bf16(w) at each owned row),
 *   grad_logits [N,E] bf16, grad_w [N,k] fp32 (may be NULL). */
int ffmoe_route_bwd(const void* go, const void* down, const int32_t* row_of,
                    const int64_t* topk_idx, const float* topk_w,
                    const void* logits, const float* lse, const int32_t* counts,
                    const float* g_aux, const float* g_z, float aux_coeff,
                    float z_coeff, int64_t N, int D, int E, int k, int gating,
                    int capacity_mode, void* wgo, void* grad_logits,
                    float* grad_w, void* stream);

/* ffmoe_route_bwd plus the aux-loss gradient through the routing weights,
 * which the reference's slow routing path makes differentiable (softmax
 * gating with expert_bias, pre_softmax, scoring_factor or n_group:
 * fused_moe.py:144-200, :1165-1189).  aux_topk_idx / aux_counts: the aux
 * loss's own routing (it differs from the dispatch routing under input
 * jitter) or NULL for the dispatch routing; logits and lse must then be the
 * un-jittered ones.  pre_softmax / scoring_factor as in ffmoe_route_fwd_ex. */
int ffmoe_route_bwd_ex(const void* go, const void* down, const int32_t* row_of,
                       const int64_t* topk_idx, const float* topk_w,
                       const void* logits, const float* lse, const int32_t* counts,
                       const float* g_aux, const float* g_z, float aux_coeff,
                       float z_coeff, int64_t N, int D, int E, int k, int gating,
                       int capacity_mode, int aux_through_weights,
                       const int64_t* aux_topk_idx, const int32_t* aux_counts,
                       int pre_softmax, float scoring_factor, void* wgo,
                       void* grad_logits, float* grad_w, void* stream);

/* Standalone GLU kernels (the reference's `activation_forward` /
 * `activation_backward`, activations.py:145-231).  up [M, 2H] bf16 ->
 * act [M, H]; grad_act [M, H], up [M, 2H] -> grad_up [M, 2H]. */
int ffmoe_glu_fwd(const void* up, int64_t M, int H, int activation, void* act,
                  void* stream);
int ffmoe_glu_bwd(const void* grad_act, const void* up, int64_t M, int H,
                  int activation, void* grad_up, void* stream);

/* Padded-layout scatter for the reference's `fused_routing_scatter` and
 * `fused_weighted_scatter` boundaries: dst[dst_row[j]] = src[j / k] * w[j]
 * (w = bf16(topk_w) or 1 when NULL) for every j with dst_row[j] >= 0.
 * dst [dst_rows, D] bf16 must be pre-zeroed by the caller. */
int ffmoe_scatter_rows(const void* src, const int64_t* dst_row, const float* w,
                       int64_t n_entries, int k, int D, int64_t dst_rows,
                       void* dst, void* stream);

/* The reference's padded-layout routing scatter, for callers of its
 * kernel-level boundary (`fused_routing_scatter`, moe_ops.py:43-149): for
 * sorted position p < n_sorted, j = sorted_order[p], e = flat_ids[j],
 * rank = p - starts[e]; if rank < mt then e2b[j] = e*mt + rank and
 * out[e2b[j]] = x[j / k].  sorted_order [n_sorted], flat_ids [N*k],
 * starts [E+1] int64 (the reference's argsort / bincount / cumsum results);
 * x [N,D] bf16; out [E*mt, D] bf16 and e2b [N*k] int64 must be zeroed by the
 * caller (entries of rank >= mt keep e2b = 0, as in the reference). */
int ffmoe_routing_scatter_padded(const int64_t* sorted_order, const int64_t* flat_ids,
                                 const int64_t* starts, const void* x, int64_t N, int D,
                                 int E, int64_t mt, int k, int64_t n_sorted, void* out,
                                 int64_t* e2b, void* stream);

/* ---------------------------------------------------------------------
 * fp32 / fp64 compute path.  The reference computes in the input dtype when
 * autocast is off (fused_moe.py:93-97, :318-327): its products are torch.bmm
 * / matmul in that dtype, its Triton kernels compute in fp32 from operands
 * of that dtype and store that dtype.  These entry points take the dtype
 * (FFMOE_DTYPE_F32 / FFMOE_DTYPE_F64) and operands of it; routing tensors
 * (topk_w, lse, logits handed to routing) stay fp32 as in the reference.
 * Accumulation is fp32 for FFMOE_DTYPE_F32 and fp64 for FFMOE_DTYPE_F64.
 * ------------------------------------------------------------------- */

/* C [M,N] (row stride ldc) = op(A) op(B), op(X) = X or X^T of a row-major X
 * with row stride ldX: the gate logits x gate^T (fused_moe.py:334, with
 * out_f32 = 1: fp32 logits for routing, the reference's logits.float()),
 * gl gate and gl^T x (:590-591), and the shared expert's products
 * (nn.py:31-40).  out_f32 = 0: C has the dtype. */
int ffmoe_t_gemm_dense(int dtype, int trans_a, int trans_b, const void* a, const void* b, void* c,
                       int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc, int out_f32,
                       void* stream);

/* Grouped rows: for each expert e, rows offsets[e]..offsets[e+1] of
 * a [rows, K] times B[e] into c [rows, N]; b_kn = 0: B[e] is [N, K] (the
 * up and down bmm's x w^T, fused_moe.py:435, :441), b_kn = 1: B[e] is
 * [K, N] (the dgrad bmm's g w, :547, :553).  tile_offsets: the route scan's
 * row-tile offsets for a 64-row tile (ffmoe_route_scan gemm_bm = 64). */
int ffmoe_t_gemm_rows(int dtype, const void* a, const void* b, const int32_t* offsets,
                      const int32_t* tile_offsets, int E, int64_t max_rows, int K, int N, int b_kn,
                      void* c, void* stream);

/* Grouped K: c[e] [M, Nc] = a[rows e]^T b[rows e] (the wgrad bmm's,
 * fused_moe.py:564-565). */
int ffmoe_t_gemm_wgrad(int dtype, const void* a, const void* b, const int32_t* offsets, int E, int M,
                       int Nc, void* c, void* stream);

/* GLU forward / backward over up [M, 2H] (activations.py:27-231).
 * compute_in_dtype = 0: fp32 math (the routed experts' Triton kernels);
 * 1: math in the dtype (the shared expert's torch ops, nn.py:33-38). */
int ffmoe_t_glu_fwd(int dtype, const void* up, int64_t M, int H, int activation,
                    int compute_in_dtype, void* out, void* stream);
int ffmoe_t_glu_bwd(int dtype, const void* grad_act, const void* up, int64_t M, int H,
                    int activation, int compute_in_dtype, void* grad_up, void* stream);

/* ffmoe_permute for rows of the dtype (moe_ops.py:43-149). */
int ffmoe_t_permute(int dtype, const void* x, const int64_t* topk_idx, float* topk_w,
                    const int32_t* offsets, const int32_t* counts, int64_t N, int D, int E,
                    int k, int mt, int capacity_mode, void* workspace, void* x_sorted,
                    int32_t* row_of, void* stream);

/* ffmoe_combine for the dtype: fp32 slot-order sum of w * rows (topk_w
 * NULL: unweighted), stored in the dtype, then + addend (may be NULL) in
 * the dtype (moe_ops.py:156-241, fused_moe.py:556-561, :590). */
int ffmoe_t_combine(int dtype, const void* rows, const int32_t* row_of, const float* topk_w,
                    const void* addend, int64_t N, int D, int k, void* out, void* stream);

/* ffmoe_route_bwd_ex for the dtype: grad_out, down, wgo and grad_logits in
 * the dtype, logits fp32 (fused_moe.py:527-591, moe_ops.py:248-332). */
int ffmoe_t_route_bwd(int dtype, const void* grad_out, const void* down, const int32_t* row_of,
                      const int64_t* topk_idx, const float* topk_w, const float* logits,
                      const float* lse, const int32_t* counts, const float* g_aux, const float* g_z,
                      float aux_coeff, float z_coeff, int64_t N, int D, int E, int k, int gating,
                      int capacity_mode, int aux_through_weights, const int64_t* aux_idx,
                      const int32_t* aux_counts, int pre_softmax, float scoring_factor, void* wgo,
                      void* grad_logits, float* grad_topk_w, void* stream);

/* The kernel-level boundary's padded scatters for the dtype: the routing
 * scatter (a row copy, ffmoe_routing_scatter_padded) and the weighted
 * scatter dst[dst_row[j]] = src[j / k] * w[j] computed in fp32
 * (ffmoe_scatter_rows; moe_ops.py:43-149, :248-332). */
int ffmoe_t_routing_scatter_padded(int dtype, const int64_t* sorted_order, const int64_t* flat_ids,
                                   const int64_t* starts, const void* x, int64_t N, int D, int E,
                                   int64_t mt, int k, int64_t n_sorted, void* out, int64_t* e2b,
                                   void* stream);
int ffmoe_t_scatter_rows(int dtype, const void* src, const int64_t* dst_row, const float* w,
                         int64_t n_entries, int k, int D, int64_t dst_rows, void* dst, void* stream);

/* ffmoe_route_fwd_ex's routing on fp32 logits [N, E] (the reference's
 * top-k reads logits.float(), fused_topk.py:52; its losses use
 * logits.float(), fused_moe.py:1179-1192): same options, no jitter (the
 * caller jitters the gate product's input). */
int ffmoe_route_logits_f32(const float* logits, const float* expert_bias, int pre_softmax,
                           float scoring_factor, int n_group, int topk_group, int64_t N, int E,
                           int k, int gating, int need_sigmoid_sum, int64_t* topk_idx,
                           float* topk_w, float* lse, void* workspace, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FFMOE_H */
