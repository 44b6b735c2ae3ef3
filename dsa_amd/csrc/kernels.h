// Internal interface between the C ABI (abi.cpp) and the gfx950 kernels
// (sparse_mla_fwd.hip, merge.hip).  Not installed; the public surface is
// include/dsa_mi355x.h.
#pragma once
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "../../include/dsa_mi355x.h"

namespace dsa {

// Everything one launch of the main kernel needs, passed by value as the
// kernel argument block.
struct FwdParams {
    const uint16_t* q;       // [tokens, H, 512] bf16
    const uint16_t* kv;      // [B, L, 512] bf16, or a [kv_rows, 512] pool when paged
    const uint16_t* q_rope;  // [tokens, H, 64] bf16
    const uint16_t* k_rope;  // [B, L, 64] bf16, or a [kv_rows, 64] pool when paged
    const int32_t* idx;      // [tokens, TOPK] int32
    uint16_t* out;           // [tokens, H, 512] bf16        (nsplit == 1)
    float* out_max;          // [tokens, H]                  (nsplit == 1)
    float* out_sum;          // [tokens, H]                  (nsplit == 1)
    float* part_o;           // [tokens, nsplit, H, 512]     (nsplit > 1)
    float* part_m;           // [tokens, nsplit, H]          (nsplit > 1)
    float* part_l;           // [tokens, nsplit, H]          (nsplit > 1)
    int B, SQ, H, L, TOPK;
    float score_scale_log2;  // softmax scale * log2(e) (the reference fixes the scale at 1/24)
    // Paged kv (NULL block_table: contiguous [B, L] rows).  Row I of batch b
    // is pool row block_table[b * max_blocks + I / block_size] * block_size
    // + I % block_size; kv and k_rope are then pools of kv_rows rows.
    const int32_t* block_table;
    int block_size, max_blocks;
    int num_blocks;          // blocks in the pool (paged); a block entry outside [0, num_blocks) masks its slots
    int kv_rows;             // rows one gather may address: L (contiguous) or the pool size
    int kv_fp8;              // 1: kv holds 656-byte fp8 rows (k_rope unused), narrow variants only
    // Non-NULL (nsplit in [2, 16], narrow variants): one arrival counter per
    // (token, head group), zero on entry; the workgroup that arrives last
    // merges the group's partials into out/out_max/out_sum and zeroes its
    // counter again.  NULL: the partials are left for the merge kernel.
    uint32_t* arrivals;
    int nsplit;              // KV splits per (token, head group)
    int ntiles;              // ceil(TOPK / tile_rows)
    int hgroups;             // H / heads_per_group
    int rowgroups;           // tokens * nsplit
};

// A validated forward call (abi.cpp: fwd_prepare), ready to enqueue.
struct FwdCall {
    FwdParams p;
    dsa_plan plan;
    bool split, fused, with_merge;
    int64_t part_rows;  // rows of the split partials (B * SQ * split * H; 0 without a split)
};

// Bytes the split partials of `rows` rows take in the scratch layout
// (part_o, part_m, part_l, each 256-byte aligned).
int64_t scratch_partial_bytes(int64_t rows);

// Validate a forward call and resolve its plan (nothing is enqueued); see
// abi.cpp.  scratch_cap > 0: the partials will come from the library's
// scratch of that many bytes (part_* must be NULL).
int fwd_prepare(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope, const uint16_t* k_rope,
                const int32_t* idx, uint16_t* out, float* out_max, float* out_sum, float* part_o, float* part_m,
                float* part_l, int B, int SQ, int H, int L, int TOPK, const dsa_fwd_options* opts,
                const dsa_plan* plan, bool with_merge, int64_t scratch_cap, FwdCall* call);

// Enqueue a prepared call; returns the ABI status (0, or a hipError_t with
// dsa_last_error set).
int fwd_enqueue(const FwdCall& call, hipStream_t stream);

// Set dsa_last_error to fmt (one %s: detail) and return code.
int set_error(int code, const char* fmt, const char* detail);

// Kernel variants compiled into the library, keyed by
// (heads_per_group, kv_waves, tile_rows, stages, mfma, pv_cols).
bool fwd_variant_exists(int heads_per_group, int kv_waves, int tile_rows, int stages, int mfma, int pv_cols);

// Slots of the index cache of one workgroup of a variant (DSA_IDX_CAP, or
// half of it where the LDS holds more per tile).
int fwd_index_cap(int heads_per_group, int pv_cols);

// Grid size (workgroups) of the main kernel for these params/plan.
int64_t fwd_grid(const FwdParams& p);

// Enqueue the main kernel; returns a hipError_t.
int launch_fwd(const FwdParams& p, int heads_per_group, int kv_waves, int tile_rows,
               int stages, int mfma, int pv_cols, hipStream_t stream);

// Largest TOPK the row bucketing handles (its LDS holds one row).
constexpr int kBucketMaxTopk = 4096;

// Enqueue the row bucketing of `tokens` index rows of `topk` entries: each
// row stably partitioned by x >> bucket_shift(kv_len) for 0 <= x < kv_len,
// every other entry last; returns a hipError_t.  topk in [1, kBucketMaxTopk],
// kv_len >= 1; out may not alias idx.
int launch_bucket_rows(const int32_t* idx, int32_t* out, int64_t tokens, int topk, int kv_len, hipStream_t stream);

// The least shift with (kv_len - 1) >> shift < 64.
int bucket_shift(int kv_len);

// Enqueue the split merge; returns a hipError_t.
int launch_merge(const float* part_o, const float* part_m, const float* part_l,
                 uint16_t* out, float* out_max, float* out_sum,
                 int tokens, int H, int nsplit, hipStream_t stream);

// Enqueue the W_UV projection of a bf16 latent output (project_uv.hip);
// returns a hipError_t.
int launch_project_uv(const uint16_t* lat, const uint16_t* w, int64_t w_head_stride, uint16_t* out_v,
                      int tokens, int H, int dv, hipStream_t stream);

// Enqueue the split merge fused with the W_UV projection; returns a hipError_t.
int launch_merge_uv(const float* part_o, const float* part_m, const float* part_l, const uint16_t* w,
                    int64_t w_head_stride, uint16_t* out_v, float* out_max, float* out_sum, int tokens,
                    int H, int nsplit, int dv, hipStream_t stream);

}  // namespace dsa

namespace dsa {

// Lightning indexer (the token selector in front of the sparse attention).
struct IndexerParams {
    const uint16_t* q;       // [B, SQ, HI, 128] bf16 indexer queries
    const uint16_t* k;       // [B, L, 128] bf16 indexer keys
    const float* w;          // [B, SQ, HI] head weights
    const int32_t* len;      // [B, SQ] candidate keys per query (keys [0, len) are candidates)
    float* logits;           // [B, SQ, L] fp32; defined for s < len
    int B, SQ, HI, L;
    int ks;                  // waves sharing a query, splitting each key stage (1, 2, 4)
    int tgroups;             // query groups per batch: ceil(SQ / (256 / HI / ks))
    int ntiles;              // key stages: ceil(L / (64 * ks))
    int tiles_per_wg;        // key stages per workgroup
};

// Enqueue the logits kernel (HI = 32 or 64, ks = 1, 2, 4); returns a hipError_t.
int launch_indexer_logits(const IndexerParams& p, hipStream_t stream);

// Enqueue the top-k selection: per row, the TOPK keys of largest logit among
// s < len (ties: lower s first), written in ascending s order, -1 padded.
int launch_indexer_topk(const float* logits, const int32_t* len, int32_t* indices, int rows, int L, int topk,
                        hipStream_t stream);

// Workspace bytes of the segmented selection (several workgroups per row, for
// few rows); 0 when rows are too many for it to pay.
int64_t indexer_topk_ws_bytes(int rows, int L);

// The same selection, segmented: three launches over the workspace (any
// contents on entry).
int launch_indexer_topk_seg(const float* logits, const int32_t* len, int32_t* indices, void* ws, int rows, int L,
                            int topk, hipStream_t stream);

}  // namespace dsa
