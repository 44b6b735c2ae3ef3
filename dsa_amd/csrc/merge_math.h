// FP32 arithmetic of the split merge (reference: dsa/merge.py:1-5, 56-91),
// shared by the merge kernel (merge.hip) and the in-kernel merge of the main
// kernel's last-arriving workgroup (sparse_mla_fwd.hip), so that the two paths
// produce identical bits:
//
//   m   = max_s m_s                          (fmaxf, from -FLT_MAX)
//   w_s = exp(m_s - m)                       (one v_exp_f32 of (m_s - m) * log2 e)
//   l   = sum_s w_s * l_s                    (fused multiply-adds, s ascending)
//   u   = sum_s w_s * u_s                    (fused multiply-adds, s ascending)
//   out = bf16(u / l)                        (IEEE division, round to nearest even)
//
// Splits are folded in ascending order and only live splits are added (an
// added zero term could turn a -0 sum into +0).
#pragma once
#include <float.h>

namespace dsa {

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float merge_f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 merge_bf16x4;

constexpr float kMergeLog2e = 1.4426950408889634f;

__device__ __forceinline__ float merge_weight(float m_s, float m) {
    return __builtin_amdgcn_exp2f((m_s - m) * kMergeLog2e);
}

__device__ __forceinline__ void merge_add(float w, float l_s, merge_f32x4 u_s, float& l, merge_f32x4& acc) {
    l = __builtin_fmaf(w, l_s, l);
    acc[0] = __builtin_fmaf(w, u_s[0], acc[0]);
    acc[1] = __builtin_fmaf(w, u_s[1], acc[1]);
    acc[2] = __builtin_fmaf(w, u_s[2], acc[2]);
    acc[3] = __builtin_fmaf(w, u_s[3], acc[3]);
}

// Column-only accumulation (the sum l is folded once per head elsewhere).
__device__ __forceinline__ void merge_add_cols(float w, merge_f32x4 u_s, merge_f32x4& acc) {
    acc[0] = __builtin_fmaf(w, u_s[0], acc[0]);
    acc[1] = __builtin_fmaf(w, u_s[1], acc[1]);
    acc[2] = __builtin_fmaf(w, u_s[2], acc[2]);
    acc[3] = __builtin_fmaf(w, u_s[3], acc[3]);
}

// Split partials folded per batch of kMergeBatch: with nsplit <= kMergeBatch
// the merge is one load round trip and exactly the formula above; later
// batches fold in with a rescale by exp(m_old - m_new).  A caller that knows
// nsplit <= BATCH < kMergeBatch may use the narrower BATCH: one batch either
// way, the same operations (the max is exact, dead slots are -FLT_MAX and
// never added), so the same bits.
constexpr int kMergeBatch = 16;

// The merge of NU (token, head) rows at 4 columns each: row r's partials are
// part_o[(base[r] + s * H) * 512 + col[r] .. + 3], part_m / part_l[base[r] + s * H]
// for s < nsplit.  Every load of a batch is issued before any arithmetic.
// Returns the unnormalised sums in acc, with m and l.
template <int NU, int BATCH = kMergeBatch>
__device__ __forceinline__ void merge_units(const float* __restrict__ part_o, const float* __restrict__ part_m,
                                            const float* __restrict__ part_l, const int64_t (&base)[NU],
                                            const int (&col)[NU], int H, int nsplit, merge_f32x4 (&acc)[NU],
                                            float (&m)[NU], float (&l)[NU]) {
#pragma unroll
    for (int r = 0; r < NU; ++r) {
        m[r] = -FLT_MAX;
        l[r] = 0.f;
        acc[r] = merge_f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int s0 = 0; s0 < nsplit; s0 += BATCH) {
        merge_f32x4 u[NU][BATCH];
        float ms[NU][BATCH], ls[NU][BATCH];
#pragma unroll
        for (int r = 0; r < NU; ++r)
#pragma unroll
            for (int j = 0; j < BATCH; ++j) {
                const bool live = s0 + j < nsplit;
                const int64_t row = base[r] + (int64_t)(live ? s0 + j : 0) * H;
                ms[r][j] = live ? part_m[row] : -FLT_MAX;
                ls[r][j] = live ? part_l[row] : 0.f;
                u[r][j] = live ? *reinterpret_cast<const merge_f32x4*>(part_o + row * 512 + col[r])
                               : merge_f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int r = 0; r < NU; ++r) {
            float mb = m[r];
#pragma unroll
            for (int j = 0; j < BATCH; ++j) mb = fmaxf(mb, ms[r][j]);
            if (s0 > 0) {
                const float alpha = merge_weight(m[r], mb);
                l[r] *= alpha;
                acc[r] *= alpha;
            }
            m[r] = mb;
#pragma unroll
            for (int j = 0; j < BATCH; ++j)
                if (s0 + j < nsplit) merge_add(merge_weight(ms[r][j], m[r]), ls[r][j], u[r][j], l[r], acc[r]);
        }
    }
}

// merge_units for NU column groups of ONE row: the row's max, weights and sum
// are computed once and applied to every group -- per value the operations
// of merge_units, so the same bits, with 1 / NU of its m / l loads and
// exponentials.
template <int NU, int BATCH = kMergeBatch>
__device__ __forceinline__ void merge_row(const float* __restrict__ part_o, const float* __restrict__ part_m,
                                          const float* __restrict__ part_l, int64_t base, const int (&col)[NU],
                                          int H, int nsplit, merge_f32x4 (&acc)[NU], float& m, float& l) {
    m = -FLT_MAX;
    l = 0.f;
#pragma unroll
    for (int r = 0; r < NU; ++r) acc[r] = merge_f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < nsplit; s0 += BATCH) {
        merge_f32x4 u[NU][BATCH];
        float ms[BATCH], ls[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const bool live = s0 + j < nsplit;
            const int64_t row = base + (int64_t)(live ? s0 + j : 0) * H;
            ms[j] = live ? part_m[row] : -FLT_MAX;
            ls[j] = live ? part_l[row] : 0.f;
#pragma unroll
            for (int r = 0; r < NU; ++r)
                u[r][j] = live ? *reinterpret_cast<const merge_f32x4*>(part_o + row * 512 + col[r])
                               : merge_f32x4{0.f, 0.f, 0.f, 0.f};
        }
        float mb = m;
#pragma unroll
        for (int j = 0; j < BATCH; ++j) mb = fmaxf(mb, ms[j]);
        if (s0 > 0) {
            const float alpha = merge_weight(m, mb);
            l *= alpha;
#pragma unroll
            for (int r = 0; r < NU; ++r) acc[r] *= alpha;
        }
        m = mb;
#pragma unroll
        for (int j = 0; j < BATCH; ++j)
            if (s0 + j < nsplit) {
                const float w = merge_weight(ms[j], m);
                l = __builtin_fmaf(w, ls[j], l);
#pragma unroll
                for (int r = 0; r < NU; ++r) merge_add_cols(w, u[r][j], acc[r]);
            }
    }
}

__device__ __forceinline__ merge_bf16x4 merge_finish(merge_f32x4 acc, float l) {
    merge_bf16x4 o;
    o[0] = (__bf16)(acc[0] / l);
    o[1] = (__bf16)(acc[1] / l);
    o[2] = (__bf16)(acc[2] / l);
    o[3] = (__bf16)(acc[3] / l);
    return o;
}

}  // namespace dsa
