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

__device__ __forceinline__ merge_bf16x4 merge_finish(merge_f32x4 acc, float l) {
    merge_bf16x4 o;
    o[0] = (__bf16)(acc[0] / l);
    o[1] = (__bf16)(acc[1] / l);
    o[2] = (__bf16)(acc[2] / l);
    o[3] = (__bf16)(acc[3] / l);
    return o;
}

}  // namespace dsa
