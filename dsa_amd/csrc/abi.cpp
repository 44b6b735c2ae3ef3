// C ABI of the library (include/dsa_mi355x.h): argument checks, launch
// planning and the main + merge launch sequence of one forward call.
//
// Reference behaviour mirrored: dsa/api.py:18-38 (input contract),
// dsa/api.py:41-60 (tuning checks), dsa/api.py:101-128 (allocation and the
// main-kernel + merge launch pair).  The ABI never throws and never allocates.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/dsa_mi355x.h"
#include "kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(int err, const char* what) {
    return fail(err, "%s: %s (hipError_t %d)", what, hipGetErrorString((hipError_t)err), err);
}


int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Largest split the in-kernel merge handles (its per-head weights are held in
// registers, one per split).
constexpr int kMaxFusedSplit = 16;

int check_shape(int B, int SQ, int H, int L, int TOPK) {
    if (B <= 0 || SQ <= 0 || H <= 0 || L <= 0 || TOPK <= 0)
        return fail(-1, "all of B, SQ, H, L, TOPK must be positive (got %d, %d, %d, %d, %d)", B, SQ, H, L, TOPK);
    if (H % 16 != 0) return fail(-1, "H must be a multiple of 16 (got %d)", H);
    // k_rope rows of one batch are addressed with 32-bit byte offsets
    if (L >= (1 << 25)) return fail(-1, "L must be below 33554432 (got %d)", L);
    if ((int64_t)B * SQ > (int64_t)1 << 30) return fail(-1, "B*SQ too large");
    return 0;
}

}  // namespace

extern "C" {

int dsa_version(void) { return (1 << 16) | 2; }

const char* dsa_last_error(void) { return g_err; }

int dsa_plan_check(const dsa_plan* plan, int B, int SQ, int H, int L, int TOPK) {
    if (!plan) return fail(-1, "plan is NULL");
    if (int rc = check_shape(B, SQ, H, L, TOPK)) return rc;
    const int hpg = plan->heads_per_group, bn = plan->tile_rows, split = plan->split, mfma = plan->mfma;
    if (mfma != 16 && mfma != 32) return fail(-1, "mfma must be 16 or 32 (got %d)", mfma);
    if (hpg <= 0 || hpg % mfma)
        return fail(-1, "heads_per_group must be a positive multiple of mfma=%d (got %d)", mfma, hpg);
    if (H % hpg) return fail(-1, "heads_per_group %d must divide H=%d", hpg, H);
    if (bn != 32 && bn != 64) return fail(-1, "tile_rows must be 32 or 64 (got %d)", bn);
    const int pv_cols = plan->pv_cols == 0 ? 512 : plan->pv_cols;
    if (pv_cols != 512 && pv_cols != 128) return fail(-1, "pv_cols must be 0 (= 512), 512 or 128 (got %d)", pv_cols);
    if (pv_cols == 512 && plan->kv_waves * (hpg / mfma) != 4)
        return fail(-1, "kv_waves * heads_per_group / mfma must be 4 (got kv_waves=%d)", plan->kv_waves);
    if (!dsa::fwd_variant_exists(hpg, plan->kv_waves, bn, plan->stages, mfma, pv_cols))
        return fail(-1,
                    "no kernel variant for heads_per_group=%d kv_waves=%d tile_rows=%d stages=%d mfma=%d pv_cols=%d",
                    hpg, plan->kv_waves, bn, plan->stages, mfma, pv_cols);
    const int ntiles = ceil_div(TOPK, bn);
    if (split < 1 || split > ntiles)
        return fail(-1, "split must be in [1, %d] for TOPK=%d (got %d)", ntiles, TOPK, split);
    const int cap = dsa::fwd_index_cap(hpg, pv_cols);
    if (ceil_div(ntiles, split) * bn > cap)
        return fail(-1, "split %d leaves more than %d slots per workgroup (TOPK=%d)", split, cap, TOPK);
    if (plan->fused_merge != 0 && plan->fused_merge != 1)
        return fail(-1, "fused_merge must be 0 or 1 (got %d)", plan->fused_merge);
    if (plan->fused_merge && (mfma != 16 || split > kMaxFusedSplit || (pv_cols == 128 && hpg != 16)))
        return fail(-1,
                    "fused_merge needs a narrow plan (mfma 16; with pv_cols 128, 16 heads per group) with split <= %d "
                    "(got mfma=%d split=%d heads_per_group=%d pv_cols=%d)",
                    kMaxFusedSplit, mfma, split, hpg, pv_cols);
    g_err[0] = 0;
    return 0;
}

}  // extern "C"

namespace {

// The planner behind dsa_plan_for; `fp8` restricts it to the variants that
// read 656-byte fp8 kv rows (the narrow ones) and prices their gathers and
// per-tile expansion; `fuse` lets it price the in-kernel merge for narrow
// plans with split <= kMaxFusedSplit.
int plan_impl(int B, int SQ, int H, int L, int TOPK, int num_cus, bool fp8, bool fuse, int64_t max_partial_bytes,
              dsa_plan* out) {
    if (!out) return fail(-1, "out is NULL");
    if (int rc = check_shape(B, SQ, H, L, TOPK)) return rc;
    if (num_cus <= 0) return fail(-1, "num_cus must be positive (got %d)", num_cus);
    // Every (variant, split) the kernels support is scored with a cost model
    // fitted to MI355X measurements, and the cheapest is taken.  One
    // workgroup (152 KiB of LDS) runs per CU, so workgroups beyond the CU
    // count run in further rounds.  Per workgroup: a prologue (index load,
    // first gather), a cost per tile, and an epilogue (row-wave merge and
    // partial stores); the gathered rows are also bounded by the HBM rate the
    // active CUs reach; a split adds the merge kernel, bounded by its
    // parallelism, or -- merged in the kernel -- a tail in which the last
    // workgroup of each group reads the group's partials back on one CU
    // (measured ≈30 GB/s: C3's 64 KiB groups cost ≈0.4 µs over the main
    // kernel, C1's and C2's 512 KiB groups 17-18 µs).
    // The column-split PV variants (pv_cols 128) replace narrow<2,2> and
    // narrow<1,4> on bf16 rows: measured 2-15 % faster on every shape swept
    // (no row-wave exchange in the epilogue); fp8 rows are read by the
    // narrow variants only.  The ping-pong variant (128 heads, pv_cols 128)
    // measured 8 % under wide<4,1> per tile on the 4096- and 32768-token
    // prefills.  The specialised-wave variants (32-row tiles, gather waves)
    // measured within ±9 % of the column-split ones, ahead where a workgroup
    // holds 32 heads.
    struct Variant {
        int hpg, kvw, bn, stages, mfma, pv_cols;
        bool bf16, fp8;
        double tile_cycles, epilogue_cycles;
    };
    static const Variant kVariants[] = {
        {128, 1, 32, 4, 32, 512, true, false, 4400.0, 18000.0},  // wide<4,1,32,4>
        {64, 2, 64, 2, 32, 512, true, false, 5000.0, 15000.0},   // wide<2,2,64,2>
        {64, 1, 64, 2, 16, 512, true, true, 7000.0, 6000.0},     // narrow<4,1>
        {32, 2, 64, 2, 16, 512, false, true, 4000.0, 10000.0},   // narrow<2,2>
        {16, 4, 64, 2, 16, 512, false, true, 2800.0, 10000.0},   // narrow<1,4>
        {32, 4, 64, 2, 16, 128, true, false, 3800.0, 6000.0},    // xp<2>: 32 heads, column-split PV
        {16, 4, 64, 2, 16, 128, true, false, 2700.0, 4000.0},    // xp<1>: 16 heads, column-split PV
        {128, 1, 32, 4, 16, 128, true, false, 4000.0, 18000.0},  // ping-pong: 128 heads, eight waves
        {32, 2, 32, 4, 16, 128, true, false, 1850.0, 6000.0},    // xs<2>: 32 heads, specialised waves
        {16, 2, 32, 4, 16, 128, true, false, 1400.0, 4000.0},    // xs<1>: 16 heads, specialised waves
    };
    constexpr double kClockMHz = 2200.0, kPrologueCycles = 9000.0, kLaunchUs = 2.0;
    constexpr double kHbmBytesPerUs = 4.8e6, kCuBytesPerUs = 3.0e4;                // sustained gather rates
    constexpr double kMergeUs = 2.0, kMergeWgBytesPerUs = 4.2e4, kMergeBytesPerUs = 6.0e6;
    constexpr double kFp8TileCycles = 1200.0;  // expanding a 64-row fp8 tile to bf16 in LDS
    constexpr double kFusedUs = 0.5, kFusedBytesPerUs = 3.0e4;  // in-kernel merge: count-in, one CU's read rate
    const int64_t tokens = (int64_t)B * SQ;
    const double gathered = (double)tokens * TOPK * (fp8 ? 656.0 : 1152.0);
    double best = -1.0;
    dsa_plan p{};
    for (const Variant& v : kVariants) {
        if (H % v.hpg) continue;
        if (fp8 ? !v.fp8 : !v.bf16) continue;
        const double tile_cycles = v.tile_cycles + (fp8 ? kFp8TileCycles : 0.0);
        const int ntiles = ceil_div(TOPK, v.bn);
        const int min_split = ceil_div(ntiles * v.bn, dsa::fwd_index_cap(v.hpg, v.pv_cols));
        const int64_t groups = tokens * (H / v.hpg);
        for (int split = min_split; split <= ntiles; ++split) {
            const int64_t wgs = groups * split;
            if (wgs > 0x7fffffff) break;
            if (max_partial_bytes > 0 && split > 1 &&
                dsa::scratch_partial_bytes(tokens * split * H) > max_partial_bytes)
                break;  // larger splits need more partials still
            const double rounds = (double)((wgs + num_cus - 1) / num_cus);
            const double tiles = (double)ceil_div(ntiles, split);
            const double wg_us = (kPrologueCycles + tiles * tile_cycles + v.epilogue_cycles) / kClockMHz;
            const double active = (double)(wgs < num_cus ? wgs : num_cus);
            const double hbm = active * kCuBytesPerUs < kHbmBytesPerUs ? active * kCuBytesPerUs : kHbmBytesPerUs;
            double main_us = rounds * wg_us;
            if (gathered / hbm > main_us) main_us = gathered / hbm;
            double merge_us = 0.0;
            if (split > 1) {
                const double bytes = (double)tokens * split * H * 2056.0;
                const double merge_wgs = (double)tokens * ((H + 1) / 2);
                const double bw = merge_wgs * kMergeWgBytesPerUs < kMergeBytesPerUs ? merge_wgs * kMergeWgBytesPerUs
                                                                                    : kMergeBytesPerUs;
                merge_us = kMergeUs + bytes / bw;
            }
            double cost = kLaunchUs + main_us + merge_us;
            int fused = 0;
            if (fuse && split > 1 && split <= kMaxFusedSplit && v.mfma == 16 && !(v.pv_cols == 128 && v.hpg != 16)) {
                const double group_bytes = (double)split * v.hpg * 2056.0;
                const double fused_cost = kLaunchUs + main_us + kFusedUs + group_bytes / kFusedBytesPerUs;
                if (fused_cost < cost) cost = fused_cost, fused = 1;
            }
            if (best < 0.0 || cost < best * 0.999) {
                best = cost;
                p.heads_per_group = v.hpg, p.kv_waves = v.kvw, p.tile_rows = v.bn, p.stages = v.stages;
                p.mfma = v.mfma, p.split = split, p.fused_merge = fused, p.pv_cols = v.pv_cols;
            }
        }
    }
    if (best < 0.0) {
        if (max_partial_bytes > 0)
            return fail(-1, "no plan for H=%d whose split partials fit in %lld bytes", H, (long long)max_partial_bytes);
        return fail(-1, "no kernel variant for H=%d", H);
    }
    *out = p;
    return dsa_plan_check(out, B, SQ, H, L, TOPK);
}

}  // namespace

extern "C" {

int dsa_plan_for(int B, int SQ, int H, int L, int TOPK, int num_cus, dsa_plan* out) {
    return plan_impl(B, SQ, H, L, TOPK, num_cus, false, true, 0, out);
}

int dsa_plan_for_opts(int B, int SQ, int H, int L, int TOPK, int num_cus, const dsa_fwd_options* opts,
                      dsa_plan* out) {
    if (opts && opts->kv_format != DSA_KV_BF16 && opts->kv_format != DSA_KV_FP8)
        return fail(-1, "kv_format must be DSA_KV_BF16 (0) or DSA_KV_FP8 (1) (got %d)", opts->kv_format);
    return plan_impl(B, SQ, H, L, TOPK, num_cus, opts && opts->kv_format == DSA_KV_FP8, true, 0, out);
}

int dsa_partial_elems(const dsa_plan* plan, int B, int SQ, int H, int64_t* part_o_elems,
                      int64_t* part_ml_elems) {
    if (!plan || !part_o_elems || !part_ml_elems) return fail(-1, "NULL argument");
    if (B <= 0 || SQ <= 0 || H <= 0) return fail(-1, "B, SQ, H must be positive");
    const int64_t rows = plan->split > 1 ? (int64_t)B * SQ * plan->split * H : 0;
    *part_o_elems = rows * 512;
    *part_ml_elems = rows;
    g_err[0] = 0;
    return 0;
}

int dsa_merge(const float* part_o, const float* part_m, const float* part_l, uint16_t* out, float* out_max,
              float* out_sum, int tokens, int H, int split, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!part_o || !part_m || !part_l || !out || !out_max || !out_sum) return fail(-1, "NULL pointer argument");
    if (tokens <= 0 || H <= 0 || split <= 0)
        return fail(-1, "tokens, H, split must be positive (got %d, %d, %d)", tokens, H, split);
    const int rc = dsa::launch_merge(part_o, part_m, part_l, out, out_max, out_sum, tokens, H, split, stream);
    if (rc) return hip_fail(rc, "merge launch");
    g_err[0] = 0;
    return 0;
}

int dsa_bucket_indices(const int32_t* idx, int32_t* out, int tokens, int TOPK, int L, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!idx || !out) return fail(-1, "NULL pointer argument");
    if (tokens <= 0 || TOPK <= 0 || L <= 0)
        return fail(-1, "tokens, TOPK and L must be positive (got %d, %d, %d)", tokens, TOPK, L);
    if (TOPK > dsa::kBucketMaxTopk)
        return fail(-1, "TOPK must be at most %d here (got %d)", dsa::kBucketMaxTopk, TOPK);
    if (idx == out) return fail(-1, "out must not alias idx");
    if (((uintptr_t)idx | (uintptr_t)out) & 3) return fail(-1, "idx and out must be 4-byte aligned");
    const int rc = dsa::launch_bucket_rows(idx, out, tokens, TOPK, L, stream);
    if (rc) return hip_fail(rc, "bucket launch");
    g_err[0] = 0;
    return 0;
}

}  // extern "C"

namespace {

// Shared checks of the W_UV entry points.
int check_uv(const uint16_t* w_uv, int64_t w_head_stride, const uint16_t* out_v, int tokens, int H, int dv) {
    if (!w_uv || !out_v) return fail(-1, "NULL pointer argument");
    if (tokens <= 0 || H <= 0) return fail(-1, "tokens and H must be positive (got %d, %d)", tokens, H);
    if (dv < 64 || dv > 256 || dv % 64)
        return fail(-1, "dv must be a multiple of 64 in [64, 256] (got %d)", dv);
    if (w_head_stride < (int64_t)dv * 512 || w_head_stride % 8)
        return fail(-1, "w_head_stride must be a multiple of 8 and >= dv * 512 (got %lld)",
                    (long long)w_head_stride);
    if ((uintptr_t)w_uv & 15) return fail(-1, "w_uv must be 16-byte aligned");
    if ((uintptr_t)out_v & 7) return fail(-1, "out_v must be 8-byte aligned");
    // Workgroups: H * ceil(tokens / 16) at most, times a d-split of 4 at most;
    // 32-bit byte offsets within 32 tokens of out_v.
    if ((int64_t)H * ((tokens + 15) / 16) * 4 > INT32_MAX) return fail(-1, "tokens * H too large");
    if ((int64_t)H * dv > (1 << 24)) return fail(-1, "H * dv too large (at most 2^24)");
    return 0;
}

}  // namespace

extern "C" {

int dsa_project_uv(const uint16_t* output, const uint16_t* w_uv, int64_t w_head_stride, uint16_t* out_v,
                   int tokens, int H, int dv, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!output) return fail(-1, "NULL pointer argument");
    if (int rc = check_uv(w_uv, w_head_stride, out_v, tokens, H, dv)) return rc;
    if ((uintptr_t)output & 15) return fail(-1, "output must be 16-byte aligned");
    const int rc = dsa::launch_project_uv(output, w_uv, w_head_stride, out_v, tokens, H, dv, stream);
    if (rc) return hip_fail(rc, "project_uv launch");
    g_err[0] = 0;
    return 0;
}

int dsa_merge_uv(const float* part_o, const float* part_m, const float* part_l, const uint16_t* w_uv,
                 int64_t w_head_stride, uint16_t* out_v, float* out_max, float* out_sum, int tokens, int H,
                 int split, int dv, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!part_o || !part_m || !part_l || !out_max || !out_sum) return fail(-1, "NULL pointer argument");
    if (int rc = check_uv(w_uv, w_head_stride, out_v, tokens, H, dv)) return rc;
    if (split <= 0) return fail(-1, "split must be positive (got %d)", split);
    if ((uintptr_t)part_o & 15) return fail(-1, "part_o must be 16-byte aligned");
    const int rc = dsa::launch_merge_uv(part_o, part_m, part_l, w_uv, w_head_stride, out_v, out_max, out_sum,
                                        tokens, H, split, dv, stream);
    if (rc) return hip_fail(rc, "merge_uv launch");
    g_err[0] = 0;
    return 0;
}

}  // extern "C"

namespace dsa {

int64_t scratch_partial_bytes(int64_t rows) {
    const auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    return up(rows * 512 * 4) + 2 * up(rows * 4);
}

// Shared by every forward entry point: validate, resolve the plan and fill
// the kernel parameters; nothing is enqueued.  scratch_cap == 0: the caller
// brings the split partials (and, for the in-kernel merge, arrival counters in
// opts).  scratch_cap > 0: the partials come from the library's scratch
// (fwd_scratch.hip), so part_o/part_m/part_l must be NULL; a NULL plan is
// planned among the splits whose partials fit in scratch_cap bytes, and an
// explicit plan whose partials do not fit is rejected.
int fwd_prepare(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope, const uint16_t* k_rope,
                const int32_t* idx, uint16_t* out, float* out_max, float* out_sum, float* part_o, float* part_m,
                float* part_l, int B, int SQ, int H, int L, int TOPK, const dsa_fwd_options* opts,
                const dsa_plan* plan, bool with_merge, int64_t scratch_cap, FwdCall* call) {
    const bool fp8 = opts && opts->kv_format == DSA_KV_FP8;
    const bool scratch = scratch_cap > 0;
    if (!q || !kv || !q_rope || (!k_rope && !fp8) || !idx) return fail(-1, "NULL input pointer");
    if (int rc = check_shape(B, SQ, H, L, TOPK)) return rc;
    // Options: scale in log2 units (the default is the reference's 1/24) and
    // the paged-kv geometry.
    float scale_log2 = (float)(1.4426950408889634 / 24.0);
    const int32_t* block_table = nullptr;
    int block_size = 0, max_blocks = 0, num_blocks = 0, kv_rows = L;
    if (opts) {
        if (opts->kv_format != DSA_KV_BF16 && opts->kv_format != DSA_KV_FP8)
            return fail(-1, "kv_format must be DSA_KV_BF16 (0) or DSA_KV_FP8 (1) (got %d)", opts->kv_format);
        if (opts->reserved32) return fail(-1, "reserved option fields must be zero");
        if ((uintptr_t)opts->arrivals & 3) return fail(-1, "arrivals must be 4-byte aligned");
        if (scratch && opts->arrivals) return fail(-1, "arrivals must be NULL here: the counters are in the scratch");
        if (opts->scale != 0.0f) {
            if (!(opts->scale > 0.0f) || !std::isfinite(opts->scale))
                return fail(-1, "scale must be a positive finite number (got %g)", (double)opts->scale);
            scale_log2 = (float)((double)opts->scale * 1.4426950408889634);
        }
        if (opts->block_table) {
            block_table = opts->block_table;
            block_size = opts->block_size;
            max_blocks = opts->max_blocks;
            if (block_size <= 0 || max_blocks <= 0 || opts->num_blocks <= 0)
                return fail(-1, "block_size, max_blocks and num_blocks must be positive (got %d, %d, %d)",
                            block_size, max_blocks, opts->num_blocks);
            if ((int64_t)max_blocks * block_size != L)
                return fail(-1, "L must equal max_blocks * block_size (%d != %d * %d)", L, max_blocks, block_size);
            if ((int64_t)opts->num_blocks * block_size >= (1 << 25))
                return fail(-1, "num_blocks * block_size must be below 33554432 (got %lld)",
                            (long long)opts->num_blocks * block_size);
            if ((uintptr_t)block_table & 3) return fail(-1, "block_table must be 4-byte aligned");
            num_blocks = opts->num_blocks;
            kv_rows = num_blocks * block_size;
        }
    }
    if (scratch && (part_o || part_m || part_l))
        return fail(-1, "part_o, part_m and part_l must be NULL here: the partials are in the scratch");
    dsa_plan local{};
    if (!plan) {
        if (!with_merge) return fail(-1, "dsa_fwd_main needs an explicit plan");
        int dev = 0, cus = 0;
        int err = (int)hipGetDevice(&dev);
        if (!err) err = (int)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (err) return hip_fail(err, "querying the CU count");
        if (int rc = plan_impl(B, SQ, H, L, TOPK, cus, fp8, scratch || (opts && opts->arrivals), scratch_cap,
                               &local))
            return rc;
        plan = &local;
    } else if (int rc = dsa_plan_check(plan, B, SQ, H, L, TOPK)) {
        return rc;
    }
    if (fp8 && (plan->mfma != 16 || (plan->pv_cols != 0 && plan->pv_cols != 512)))
        return fail(-1, "fp8 kv rows need a narrow plan (mfma 16, pv_cols 512)");
    const bool split = plan->split > 1;
    const int64_t part_rows = split ? (int64_t)B * SQ * plan->split * H : 0;
    if (scratch && split && scratch_partial_bytes(part_rows) > scratch_cap)
        return fail(-1, "split=%d needs %lld bytes of split partials; the scratch holds %lld (pass a plan with a "
                    "smaller split, or NULL to plan within it, or use dsa_fwd_opts with your own buffers)",
                    plan->split, (long long)scratch_partial_bytes(part_rows), (long long)scratch_cap);
    // The in-kernel merge needs arrival counters (the caller's, or the
    // scratch's); without them the merge kernel runs (same bits).
    const bool fused = split && with_merge && plan->fused_merge && (scratch || (opts && opts->arrivals));
    if ((!split || with_merge) && (!out || !out_max || !out_sum)) return fail(-1, "NULL output pointer");
    if (split && !scratch && (!part_o || !part_m || !part_l))
        return fail(-1, "split=%d needs part_o, part_m and part_l", plan->split);
    // 16-byte vector accesses need 16-byte aligned rows.
    if (((uintptr_t)q | (uintptr_t)kv | (uintptr_t)q_rope | (uintptr_t)k_rope) & 15)
        return fail(-1, "q, kv, q_rope and k_rope must be 16-byte aligned");  // fp8 rows: 656 = 41 x 16
    if (out && ((uintptr_t)out & 15)) return fail(-1, "out must be 16-byte aligned");
    if (split && ((uintptr_t)part_o & 15)) return fail(-1, "part_o must be 16-byte aligned");
    const int64_t rowgroups = (int64_t)B * SQ * plan->split;
    if (rowgroups * (H / plan->heads_per_group) > 0x7fffffff) return fail(-1, "grid too large");

    FwdParams& p = call->p;
    p = FwdParams{};
    p.q = q;
    p.kv = kv;
    p.q_rope = q_rope;
    p.k_rope = k_rope;
    p.idx = idx;
    p.out = out;
    p.out_max = out_max;
    p.out_sum = out_sum;
    p.part_o = part_o;
    p.part_m = part_m;
    p.part_l = part_l;
    p.B = B;
    p.SQ = SQ;
    p.H = H;
    p.L = L;
    p.TOPK = TOPK;
    p.score_scale_log2 = scale_log2;
    p.block_table = block_table;
    p.block_size = block_size;
    p.max_blocks = max_blocks;
    p.num_blocks = num_blocks;
    p.kv_rows = kv_rows;
    p.kv_fp8 = fp8 ? 1 : 0;
    p.nsplit = plan->split;
    p.ntiles = ceil_div(TOPK, plan->tile_rows);
    p.hgroups = H / plan->heads_per_group;
    p.rowgroups = (int)rowgroups;
    p.arrivals = fused && !scratch ? opts->arrivals : nullptr;
    call->plan = *plan;
    call->split = split;
    call->fused = fused;
    call->with_merge = with_merge;
    call->part_rows = part_rows;
    return 0;
}

// Enqueue a prepared call: the main kernel and, when it splits and does not
// merge inside the main kernel, the merge kernel.
int fwd_enqueue(const FwdCall& c, hipStream_t stream) {
    const FwdParams& p = c.p;
    int rc = launch_fwd(p, c.plan.heads_per_group, c.plan.kv_waves, c.plan.tile_rows, c.plan.stages, c.plan.mfma,
                        c.plan.pv_cols == 0 ? 512 : c.plan.pv_cols, stream);
    if (rc) return hip_fail(rc, "main kernel launch");
    if (c.split && c.with_merge && !c.fused) {
        rc = launch_merge(p.part_o, p.part_m, p.part_l, p.out, p.out_max, p.out_sum, p.B * p.SQ, p.H, p.nsplit,
                          stream);
        if (rc) return hip_fail(rc, "merge launch");
    }
    g_err[0] = 0;
    return 0;
}

int set_error(int code, const char* fmt, const char* detail) { return fail(code, fmt, detail); }

}  // namespace dsa

namespace {

int fwd_impl(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope, const uint16_t* k_rope,
             const int32_t* idx, uint16_t* out, float* out_max, float* out_sum, float* part_o, float* part_m,
             float* part_l, int B, int SQ, int H, int L, int TOPK, const dsa_fwd_options* opts,
             const dsa_plan* plan, hipStream_t stream, bool with_merge) {
    dsa::FwdCall call;
    if (int rc = dsa::fwd_prepare(q, kv, q_rope, k_rope, idx, out, out_max, out_sum, part_o, part_m, part_l, B, SQ,
                                  H, L, TOPK, opts, plan, with_merge, 0, &call))
        return rc;
    return dsa::fwd_enqueue(call, stream);
}

}  // namespace

extern "C" {

int dsa_fwd(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope, const uint16_t* k_rope,
            const int32_t* idx, uint16_t* out, float* out_max, float* out_sum, float* part_o, float* part_m,
            float* part_l, int B, int SQ, int H, int L, int TOPK, const dsa_plan* plan, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    return fwd_impl(q, kv, q_rope, k_rope, idx, out, out_max, out_sum, part_o, part_m, part_l, B, SQ, H, L,
                    TOPK, nullptr, plan, stream, true);
}

int dsa_fwd_main(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope, const uint16_t* k_rope,
                 const int32_t* idx, uint16_t* out, float* out_max, float* out_sum, float* part_o,
                 float* part_m, float* part_l, int B, int SQ, int H, int L, int TOPK, const dsa_plan* plan,
                 void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    return fwd_impl(q, kv, q_rope, k_rope, idx, out, out_max, out_sum, part_o, part_m, part_l, B, SQ, H, L,
                    TOPK, nullptr, plan, stream, false);
}

int dsa_fwd_opts(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope, const uint16_t* k_rope,
                 const int32_t* idx, uint16_t* out, float* out_max, float* out_sum, float* part_o, float* part_m,
                 float* part_l, int B, int SQ, int H, int L, int TOPK, const dsa_fwd_options* opts,
                 const dsa_plan* plan, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    return fwd_impl(q, kv, q_rope, k_rope, idx, out, out_max, out_sum, part_o, part_m, part_l, B, SQ, H, L,
                    TOPK, opts, plan, stream, true);
}

int dsa_fwd_main_opts(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope, const uint16_t* k_rope,
                      const int32_t* idx, uint16_t* out, float* out_max, float* out_sum, float* part_o,
                      float* part_m, float* part_l, int B, int SQ, int H, int L, int TOPK,
                      const dsa_fwd_options* opts, const dsa_plan* plan, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    return fwd_impl(q, kv, q_rope, k_rope, idx, out, out_max, out_sum, part_o, part_m, part_l, B, SQ, H, L,
                    TOPK, opts, plan, stream, false);
}

}  // extern "C"

extern "C" {

int dsa_indexer_logits(const uint16_t* q_idx, const uint16_t* k_idx, const float* weights, const int32_t* lengths,
                       float* logits, int B, int SQ, int HI, int L, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!q_idx || !k_idx || !weights || !lengths || !logits) return fail(-1, "NULL pointer argument");
    if (B <= 0 || SQ <= 0 || L <= 0) return fail(-1, "B, SQ, L must be positive (got %d, %d, %d)", B, SQ, L);
    if (HI != 32 && HI != 64) return fail(-1, "indexer heads must be 32 or 64 (got %d)", HI);
    // keys of one batch are addressed with 32-bit byte offsets
    if (L >= (1 << 24)) return fail(-1, "L must be below 16777216 (got %d)", L);
    if (((uintptr_t)q_idx | (uintptr_t)k_idx) & 15) return fail(-1, "q_idx and k_idx must be 16-byte aligned");
    if (((uintptr_t)weights | (uintptr_t)lengths | (uintptr_t)logits) & 3)
        return fail(-1, "weights, lengths and logits must be 4-byte aligned");
    dsa::IndexerParams p{};
    p.q = q_idx;
    p.k = k_idx;
    p.w = weights;
    p.len = lengths;
    p.logits = logits;
    p.B = B;
    p.SQ = SQ;
    p.HI = HI;
    p.L = L;
    // Waves per query: all four share one query's 64 heads when SQ * HI <= 64
    // (decode), two when <= 128, else each wave owns its own query slot.
    p.ks = (int64_t)SQ * HI <= 64 ? 4 : ((int64_t)SQ * HI <= 128 ? 2 : 1);
    p.tgroups = ceil_div(SQ, 256 / HI / p.ks);
    p.ntiles = ceil_div(L, 64 * p.ks);
    // About 1024 / ks workgroups (a stage of ks x 16 KiB, two stages per
    // workgroup): decode spreads one query's keys over many CUs, prefill keeps
    // every key stage of a query group in one workgroup.
    const int64_t work = (int64_t)B * p.tgroups * p.ntiles;
    const int64_t target = 1024 / p.ks;
    p.tiles_per_wg = (int)((work + target - 1) / target);
    if (p.tiles_per_wg < 1) p.tiles_per_wg = 1;
    if (p.tiles_per_wg > p.ntiles) p.tiles_per_wg = p.ntiles;
    // grid.x * 256 work-items must stay below 2^32
    if ((int64_t)B * p.tgroups >= (1 << 24)) return fail(-1, "too many query groups (B * ceil(SQ * HI / 256))");
    const int rc = dsa::launch_indexer_logits(p, stream);
    if (rc) return hip_fail(rc, "indexer logits launch");
    g_err[0] = 0;
    return 0;
}

int dsa_indexer_topk(const float* logits, const int32_t* lengths, int32_t* indices, int B, int SQ, int L, int TOPK,
                     void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!logits || !lengths || !indices) return fail(-1, "NULL pointer argument");
    if (B <= 0 || SQ <= 0 || L <= 0 || TOPK <= 0)
        return fail(-1, "B, SQ, L, TOPK must be positive (got %d, %d, %d, %d)", B, SQ, L, TOPK);
    // a row's bytes are addressed by a 32-bit buffer range
    if (L >= (1 << 28)) return fail(-1, "L must be below 268435456 (got %d)", L);
    // one 1024-thread workgroup per row: rows * 1024 work-items below 2^32
    if ((int64_t)B * SQ >= (1 << 22)) return fail(-1, "B * SQ must be below 4194304 (got %lld)", (long long)B * SQ);
    const int rc = dsa::launch_indexer_topk(logits, lengths, indices, B * SQ, L, TOPK, stream);
    if (rc) return hip_fail(rc, "indexer top-k launch");
    g_err[0] = 0;
    return 0;
}

int64_t dsa_indexer_topk_ws_bytes(int B, int SQ, int L, int TOPK) {
    if (B <= 0 || SQ <= 0 || L <= 0 || TOPK <= 0 || L >= (1 << 28) || (int64_t)B * SQ >= (1 << 22)) return 0;
    return dsa::indexer_topk_ws_bytes(B * SQ, L);
}

int dsa_indexer_topk_ws(const float* logits, const int32_t* lengths, int32_t* indices, int B, int SQ, int L,
                        int TOPK, void* workspace, int64_t workspace_bytes, void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    const int64_t need = dsa_indexer_topk_ws_bytes(B, SQ, L, TOPK);
    if (!workspace || need == 0) return dsa_indexer_topk(logits, lengths, indices, B, SQ, L, TOPK, stream);
    if (!logits || !lengths || !indices) return fail(-1, "NULL pointer argument");
    if (workspace_bytes < need)
        return fail(-1, "workspace of %lld bytes is below the %lld needed", (long long)workspace_bytes,
                    (long long)need);
    if ((uintptr_t)workspace & 15) return fail(-1, "workspace must be 16-byte aligned");
    const int rc = dsa::launch_indexer_topk_seg(logits, lengths, indices, workspace, B * SQ, L, TOPK, stream);
    if (rc) return hip_fail(rc, "segmented indexer top-k launch");
    g_err[0] = 0;
    return 0;
}

}  // extern "C"
