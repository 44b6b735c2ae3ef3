/*
 * dsa_mi355x.h -- C ABI of the MI355X (gfx950) sparse-MLA attention forward.
 *
 * The library computes, for every token t = (b, s) and head h,
 *
 *   score_j = (q[t,h,:512] . kv[b,I_j,:] + q_rope[t,h,:64] . k_rope[b,I_j,:]) / 24
 *             (scale 1/24 as in the reference; dsa_fwd_opts takes another)
 *   score_j = -inf  when I_j < 0 or I_j >= L            (index masked, slot kept)
 *   max     = max_j score_j
 *   sum     = sum_j exp(score_j - max)                  (FP32 exponentials)
 *   out     = bf16( sum_j bf16(exp(score_j - max)) * kv[b,I_j,:] / sum )
 *
 * over the TOPK slots I_j = indices[t, j].  Duplicate slots keep their weight.
 * Every row needs at least one valid slot (an all-invalid row returns NaN).
 *
 * Magnitude bound.  The kernels form exp(score - m_ref) against a reference
 * max m_ref taken from the first tile and recompute a range once with the
 * exact max only when a score exceeds m_ref by more than 64 log2 units, so a
 * weight before the division by sum can reach 2^64 (the reference's never
 * exceeds 1).  A workgroup covers S <= DSA_IDX_CAP = 2048 slots, and its FP32
 * output accumulators stay finite whenever
 *   max|kv| * S < 2^128 / 2^64,  i.e. for every call  max|kv| < 2^53 (9.0e15),
 * against max|kv| * TOPK < 2^128 (3.4e38) for the FP32 reference.  Beyond the
 * bound the output may be inf or NaN; max and sum are unaffected.
 *
 * Conventions of every entry point:
 *   - plain pointers to device memory; bf16 tensors are passed as uint16_t
 *     bit patterns; all tensors dense row-major (contiguous);
 *   - the library allocates and frees nothing, and keeps no state across calls
 *     other than read-only kernel handles and, for dsa_fwd_noalloc only, its
 *     static scratch array (below);
 *   - work is enqueued on `stream`, a hipStream_t passed as void* (NULL = the
 *     default stream); no call synchronises the device.  The header needs no
 *     HIP header, so C and FFI callers include it on its own;
 *   - return value: 0 = success, < 0 = invalid argument (nothing was enqueued),
 *     > 0 = a hipError_t from the launch; dsa_last_error() then describes it.
 *     No entry point throws.
 *
 * Reference interface replaced (CHNJZ/dsa):
 *   dsa/api.py:76-132  forward()         -> dsa_plan_for + dsa_fwd (+ dsa_merge inside)
 *   dsa/api.py:115-123 workspace_attention / ragged_attention launches -> main kernel of dsa_fwd
 *   dsa/api.py:124-128 merge_partials launch (dsa/merge.py:13-91)     -> dsa_merge
 *   dsa/config.py:10-19 Tuning, dsa/api.py:41-60 _check_tuning       -> dsa_plan, dsa_plan_check
 */
#ifndef DSA_MI355X_H
#define DSA_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_HEAD_DIM 512  /* latent (kv / value) width */
#define DSA_ROPE_DIM 64   /* rotary part of the key */
#define DSA_IDX_CAP 2048  /* max TOPK slots one workgroup handles (split >= ceil(TOPK/2048)) */

/*
 * Launch plan of one call.  Replaces dsa.Tuning (dsa/config.py:10-19), whose
 * fields were Ascend-specific (BM, BN, split, direct_nz, pv_cols, share_score).
 *
 *   heads_per_group : query heads one workgroup owns; divides H
 *   tile_rows       : gathered rows per LDS ring stage (32 or 64)
 *   split           : KV splits per (token, head group); > 1 adds the FP32 merge
 *   kv_waves        : waves that share a head slice and split each tile's rows
 *                     (heads_per_group / mfma * kv_waves == 4)
 *   stages          : LDS ring depth (2 or 4)
 *   mfma            : heads per wave = MFMA block: 32 (v_mfma_f32_32x32x16_bf16;
 *                     heads_per_group 128 with tile_rows 32 and 4 stages, or 64
 *                     with kv_waves 2) or 16 (v_mfma_f32_16x16x32_bf16;
 *                     heads_per_group 64, 32 or 16; tile_rows 64, 2 stages)
 *   fused_merge     : 0 or 1.  1 (mfma 16 and split <= 16 only): the merge
 *                     runs inside the main kernel -- the last workgroup of
 *                     each (token, head group) to finish merges its partials,
 *                     one launch instead of two -- whenever the call supplies
 *                     dsa_fwd_options.arrivals; otherwise (dsa_fwd, or no
 *                     arrivals) the merge kernel runs.  Same bits either way.
 *                     No effect when split == 1.
 *   pv_cols         : output columns one wave computes in PV (the reference's
 *                     Tuning.pv_cols, dsa/config.py:10-19): 0 or 512 -- each
 *                     wave computes all 512 columns for its own rows (the
 *                     variants above) -- or 128: the four waves split each
 *                     64-row tile's rows for QK and the softmax, exchange the
 *                     bf16 P tile through LDS and split the 512 output columns
 *                     for PV (mfma 16, kv_waves 4, tile_rows 64, stages 2,
 *                     heads_per_group 16, 32 or 64; with 64 heads a workgroup
 *                     holds at most 1024 slots).
 */
typedef struct dsa_plan {
    int32_t heads_per_group;
    int32_t tile_rows;
    int32_t split;
    int32_t kv_waves;
    int32_t stages;
    int32_t mfma;
    int32_t fused_merge;
    int32_t pv_cols;
} dsa_plan;

/* Library version, (major << 16) | minor.  1.1: dsa_plan.pv_cols (a reserved
 * zero field in 1.0, which still selects the same plans) and dsa_fwd_noalloc;
 * 1.2: dsa_bucket_indices. */
int dsa_version(void);

/* Thread-local text of the last failure on this thread ("" if none). */
const char* dsa_last_error(void);

/*
 * Default plan for a shape on a device with `num_cus` compute units.
 * Replaces the shape-keyed table lookup of dsa/api.py:88-95 (_DEFAULT_CONFIGS),
 * which rejected every shape outside its 16 entries; this covers any shape the
 * kernels support.  Pure host logic: touches no device.
 */
int dsa_plan_for(int B, int SQ, int H, int L, int TOPK, int num_cus, dsa_plan* out);

/*
 * Validate a caller-supplied plan against a shape (dsa/api.py:41-60).
 * Pure host logic.
 */
int dsa_plan_check(const dsa_plan* plan, int B, int SQ, int H, int L, int TOPK);

/*
 * Partial-buffer sizes (in float elements) a plan needs; 0 when split == 1.
 * part_o: [B*SQ, split, H, 512]; part_m, part_l: [B*SQ, split, H].
 * Mirrors the allocation at dsa/api.py:110-113.
 */
int dsa_partial_elems(const dsa_plan* plan, int B, int SQ, int H,
                      int64_t* part_o_elems, int64_t* part_ml_elems);

/*
 * Sparse-MLA attention forward (dsa/api.py:76-132).
 *
 *   q      [B, SQ, H, 512] bf16     kv     [B, L, 1, 512] bf16
 *   q_rope [B, SQ, H, 64]  bf16     k_rope [B, L, 1, 64]  bf16
 *   idx    [B, SQ, 1, TOPK] int32
 *   out    [B, SQ, H, 512] bf16     out_max, out_sum [B, 1, SQ, H] fp32
 *   part_o, part_m, part_l: split partials (dsa_partial_elems); may be NULL when
 *   plan->split == 1.  With split > 1 this enqueues the main kernel and then
 *   the merge kernel on the same stream.
 *   plan: NULL selects dsa_plan_for(..., device CU count).
 */
int dsa_fwd(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope,
            const uint16_t* k_rope, const int32_t* idx,
            uint16_t* out, float* out_max, float* out_sum,
            float* part_o, float* part_m, float* part_l,
            int B, int SQ, int H, int L, int TOPK,
            const dsa_plan* plan, void* stream);

/*
 * The main kernel of dsa_fwd alone (dsa/api.py:115-123): with plan->split == 1
 * it writes out/out_max/out_sum; with split > 1 it writes only the partials
 * and the caller completes the call with dsa_merge (for example after
 * combining partials computed over different KV shards).  plan must be
 * non-NULL here.
 */
int dsa_fwd_main(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope,
                 const uint16_t* k_rope, const int32_t* idx,
                 uint16_t* out, float* out_max, float* out_sum,
                 float* part_o, float* part_m, float* part_l,
                 int B, int SQ, int H, int L, int TOPK,
                 const dsa_plan* plan, void* stream);

/*
 * Options beyond the reference's operator contract, which fixes the scale at
 * 1/24 and takes only contiguous kv (dsa/api.py:18-38, 77-86).  A
 * zero-initialised struct selects exactly the reference behaviour.
 *
 *   scale       : softmax scale applied to q.k (> 0); 0 selects 1/24 = 576^-0.5.
 *                 Models keep their own scale (e.g. (d_nope + d_rope)^-0.5).
 *   block_table : paged kv.  NULL: kv [B, L, 1, 512] and k_rope [B, L, 1, 64]
 *                 as in dsa_fwd.  Otherwise kv is a pool [num_blocks,
 *                 block_size, 1, 512], k_rope a pool [num_blocks, block_size,
 *                 1, 64], block_table is int32 [B, max_blocks], and logical
 *                 row I of batch b is pool row
 *                 block_table[b * max_blocks + I / block_size] * block_size
 *                 + I % block_size.  L must equal max_blocks * block_size and
 *                 num_blocks * block_size must be below 33554432.  Indices stay
 *                 logical and are masked as in dsa_fwd; a slot whose block
 *                 entry lies outside [0, num_blocks) is masked as well.
 *   kv_format   : DSA_KV_BF16 (0): kv and k_rope as above.  DSA_KV_FP8 (1): kv
 *                 holds 656-byte rows, [B, L, 656] bytes (or a [num_blocks,
 *                 block_size, 656] pool) -- 512 OCP float8 e4m3 latent values,
 *                 4 fp32 scales (scale i covers dims 128 i .. 128 i + 127), 64
 *                 bf16 rope values -- and k_rope is unused (may be NULL).  The
 *                 kernel computes with kv[d] = bf16(fp32(e4m3[d]) * scale[d /
 *                 128]) (both roundings to nearest even) and the rope values;
 *                 only narrow plans (mfma 16) read fp8 rows.
 *   arrivals    : NULL, or uint32 [B * SQ * (H / heads_per_group)] arrival
 *                 counters for a plan with fused_merge = 1 and split > 1 (one
 *                 per (token, head group)).  They must be zero before the
 *                 first call; every call leaves them zero again once its
 *                 kernel has completed, so one array serves any number of
 *                 calls in stream order.  Calls that can run at the same time
 *                 (other streams) need arrays of their own.  Ignored by
 *                 dsa_fwd_main_opts and by plans that do not fuse the merge.
 *   reserved32  : must be zero.
 */
#define DSA_KV_BF16 0
#define DSA_KV_FP8 1
typedef struct dsa_fwd_options {
    float scale;
    int32_t block_size;
    int32_t max_blocks;
    int32_t num_blocks;
    const int32_t* block_table;
    int32_t kv_format;
    int32_t reserved32;
    uint32_t* arrivals;
} dsa_fwd_options;

/*
 * dsa_fwd and dsa_fwd_main with options (opts NULL = all defaults).  No
 * reference counterpart: the softmax scale, paged kv and the fp8 kv row
 * format are the next steps beyond the reference's fixed-scale,
 * contiguous bf16 cache operator (dsa/api.py:30-33); the arrival counters
 * fold the reference's second launch (the merge task, dsa/api.py:124-128)
 * into the main kernel.
 */
int dsa_fwd_opts(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope,
                 const uint16_t* k_rope, const int32_t* idx,
                 uint16_t* out, float* out_max, float* out_sum,
                 float* part_o, float* part_m, float* part_l,
                 int B, int SQ, int H, int L, int TOPK,
                 const dsa_fwd_options* opts, const dsa_plan* plan, void* stream);

/*
 * dsa_plan_for for a call with options: with kv_format DSA_KV_FP8 it plans
 * among the variants that read fp8 rows (no reference counterpart; see
 * dsa_fwd_options).  Pure host logic.
 */
int dsa_plan_for_opts(int B, int SQ, int H, int L, int TOPK, int num_cus, const dsa_fwd_options* opts,
                      dsa_plan* out);

int dsa_fwd_main_opts(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope,
                      const uint16_t* k_rope, const int32_t* idx,
                      uint16_t* out, float* out_max, float* out_sum,
                      float* part_o, float* part_m, float* part_l,
                      int B, int SQ, int H, int L, int TOPK,
                      const dsa_fwd_options* opts, const dsa_plan* plan, void* stream);

/*
 * Row bucketing of the top-k indices, a pre-pass for prefill-sized calls.
 * No counterpart in the reference (which takes the slots in the caller's
 * order).
 *
 * out[t, :] (t < tokens, TOPK int32 entries each) is idx[t, :] stably
 * partitioned by kv row range: bucket x >> s for a row index 0 <= x < L,
 * where s is the least shift with (L - 1) >> s < 64, and one last bucket
 * for every other entry (-1 or out of range); buckets ascending, and within
 * a bucket the entries keep their order in idx.  A forward call on `out`
 * instead of `idx` computes the same attention (the slots' order does not
 * enter it) up to the order of its FP32 sums, and with many tokens it
 * gathers faster: the kernels gather a token's slots 64 at a time, and with
 * every token's tiles drawn from the same row ranges in the same order,
 * workgroups that run together share L2 lines.  dsa_amd.forward runs it for
 * calls of 256 tokens or more.  TOPK <= 4096; out must not alias idx.
 * Launches one kernel on `stream`; allocates nothing.
 */
int dsa_bucket_indices(const int32_t* idx, int32_t* out, int tokens, int TOPK, int L, void* stream);

/*
 * dsa_fwd_opts for callers that cannot allocate: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  No
 * counterpart in the reference.
 *
 * Same arguments and results as dsa_fwd_opts without part_o / part_m /
 * part_l: the split partials -- and the arrival counters of a plan with
 * fused_merge = 1 -- live in a static device array of the library (one per
 * GPU, held until the process ends) whose partial region is
 * DSA_NOALLOC_PARTIAL_BYTES bytes.  opts->arrivals must be NULL.  A call
 * whose partials, B * SQ * split * H * (512 + 2) * 4 bytes (each of the three
 * arrays 256-byte aligned), exceed it is rejected (< 0, nothing enqueued);
 * plan == NULL plans among the splits that fit.  The call allocates and
 * frees nothing (no hipMalloc, hipFree or allocating library routine).  The
 * first call on a GPU also enqueues one small kernel that zeroes the
 * counters.  Every call on a GPU shares that GPU's array and leaves its last
 * partials there: calls that can overlap on one GPU (other streams,
 * concurrently replayed graphs) race on it.
 */
#define DSA_NOALLOC_PARTIAL_BYTES (32 * 1024 * 1024)
int dsa_fwd_noalloc(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope,
                    const uint16_t* k_rope, const int32_t* idx,
                    uint16_t* out, float* out_max, float* out_sum,
                    int B, int SQ, int H, int L, int TOPK,
                    const dsa_fwd_options* opts, const dsa_plan* plan, void* stream);

/*
 * FP32 merge of split partials (dsa/merge.py:13-91):
 *   m = max_s m_s;  w_s = exp(m_s - m);  l = sum_s w_s l_s;
 *   out = bf16(sum_s w_s u_s / l);  out_max = m;  out_sum = l.
 *   part_o [tokens, split, H, 512], part_m/part_l [tokens, split, H] fp32.
 * A split with (m_s = -FLT_MAX, l_s = 0, u_s = 0) carries weight 0.
 */
int dsa_merge(const float* part_o, const float* part_m, const float* part_l,
              uint16_t* out, float* out_max, float* out_sum,
              int tokens, int H, int split, void* stream);

/*
 * W_UV output projection: the step after the attention (no reference
 * counterpart; the reference stops at the 512-wide latent output and leaves
 * the model's own scale and projections to the caller, README.md:81-83,
 * FAIRNESS_AUDIT.md:28).  In MLA's absorbed form each head's latent output
 * goes through that head's slice of the kv up-projection
 * (DeepSeek-V3.2-Exp inference/model.py, MLA.forward:
 * x = einsum("bshc,hdc->bshd", x, wkv_b[:, -v_head_dim:])):
 *
 *   out_v[t, h, d] = bf16( sum_{c < 512} output[t, h, c] * w_uv[h * w_head_stride + d * 512 + c] )
 *
 *   output [tokens, H, 512] bf16 (dsa_fwd's output, 16-byte aligned)
 *   w_uv   bf16 rows of 512, dv rows per head, heads w_head_stride elements
 *          apart (>= dv * 512, a multiple of 8; 16-byte aligned) -- so the
 *          value rows of wkv_b viewed as [H, d_nope + dv, 512] go in as they
 *          are, with w_head_stride = (d_nope + dv) * 512
 *   out_v  [tokens, H, dv] bf16 (8-byte aligned); dv a multiple of 64 in [64, 256]
 * FP32 accumulation, one bf16 rounding.
 */
int dsa_project_uv(const uint16_t* output, const uint16_t* w_uv, int64_t w_head_stride,
                   uint16_t* out_v, int tokens, int H, int dv, void* stream);

/*
 * dsa_merge and dsa_project_uv in one launch (no reference counterpart):
 * the merged 512-wide rows stay on chip and are never written.  out_v,
 * out_max and out_sum are bit-identical to dsa_merge followed by
 * dsa_project_uv.  part_o/part_m/part_l as for dsa_merge; w_uv, out_v, dv
 * as for dsa_project_uv.
 */
int dsa_merge_uv(const float* part_o, const float* part_m, const float* part_l,
                 const uint16_t* w_uv, int64_t w_head_stride, uint16_t* out_v,
                 float* out_max, float* out_sum, int tokens, int H, int split, int dv,
                 void* stream);

/*
 * Lightning indexer: the token selector that produces `idx` for dsa_fwd (the
 * step before the attention; no reference counterpart -- the reference takes
 * the indices as an input, README.md:19-21).
 *
 *   logits[t, s] = sum_j w[t, j] * relu(q_idx[t, j, :] . k_idx[b, s, :])   for s < len[t]
 *
 *   q_idx   [B, SQ, HI, 128] bf16 (HI = 32 or 64)   k_idx [B, L, 128] bf16
 *   weights [B, SQ, HI] fp32                        lengths [B, SQ] int32, clamped to [0, L]
 *   logits  [B, SQ, L] fp32: defined for s < lengths[t] (entries past a row's
 *           length are unspecified).
 *
 * dsa_indexer_topk: for every row, the TOPK keys s < lengths[t] of largest
 * logit (ties: lower s first), written to indices [B, SQ, 1, TOPK] in
 * ascending s order and padded with -1 -- directly the `idx` of dsa_fwd.
 * Bit-exact given the same logits.
 */
int dsa_indexer_logits(const uint16_t* q_idx, const uint16_t* k_idx, const float* weights,
                       const int32_t* lengths, float* logits,
                       int B, int SQ, int HI, int L, void* stream);

int dsa_indexer_topk(const float* logits, const int32_t* lengths, int32_t* indices,
                     int B, int SQ, int L, int TOPK, void* stream);

/*
 * dsa_indexer_topk with a workspace (no reference counterpart, like the
 * indexer).  With few rows (B * SQ <= 32) one workgroup per row leaves most
 * CUs idle; given `workspace` of at least dsa_indexer_topk_ws_bytes bytes
 * (16-byte aligned, any contents), every row is split over 8 workgroups in
 * three launches instead.  Same result bit for bit.  A NULL workspace, or a
 * size query that returns 0 (many rows), selects dsa_indexer_topk's kernel.
 */
int64_t dsa_indexer_topk_ws_bytes(int B, int SQ, int L, int TOPK);

int dsa_indexer_topk_ws(const float* logits, const int32_t* lengths, int32_t* indices,
                        int B, int SQ, int L, int TOPK, void* workspace, int64_t workspace_bytes,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_MI355X_H */
