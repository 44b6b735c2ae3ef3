// FP32 merge of split-KV partials (reference: dsa/merge.py:13-91, formula at
// dsa/merge.py:1-5):
//   m = max_s m_s;  w_s = exp(m_s - m);  l = sum_s w_s * l_s;
//   out = bf16(sum_s w_s * u_s / l);  out_max = m;  out_sum = l.
// One workgroup merges two heads of one token; each thread owns 4 of the 512
// columns and streams the split partials with 16-byte loads, kMergeBatch
// splits in flight at a time.  The arithmetic is merge_math.h's, which the
// main kernel's in-kernel merge and the merge + W_UV kernel share.
#include <hip/hip_runtime.h>
#include <float.h>
#include <stdint.h>

#include "kernels.h"
#include "merge_math.h"

namespace dsa {
namespace {

typedef merge_f32x4 f32x4;

__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ part_o,
                                                    const float* __restrict__ part_m,
                                                    const float* __restrict__ part_l,
                                                    uint16_t* __restrict__ out,
                                                    float* __restrict__ out_max,
                                                    float* __restrict__ out_sum, int H, int nsplit) {
    const int pairs = (H + 1) >> 1;
    const int token = blockIdx.x / pairs;
    const int h = (blockIdx.x % pairs) * 2 + (threadIdx.x >> 7);
    if (h >= H) return;
    const int col = (threadIdx.x & 127) * 4;
    const int64_t base[1] = {(int64_t)token * nsplit * H + h};  // + s * H
    const int cols[1] = {col};
    f32x4 acc[1];
    float m[1], l[1];
    merge_units<1>(part_o, part_m, part_l, base, cols, H, nsplit, acc, m, l);
    const int64_t orow = (int64_t)token * H + h;
    *reinterpret_cast<merge_bf16x4*>(out + orow * 512 + col) = merge_finish(acc[0], l[0]);
    if ((threadIdx.x & 127) == 0) {
        out_max[orow] = m[0];
        out_sum[orow] = l[0];
    }
}

}  // namespace

int launch_merge(const float* part_o, const float* part_m, const float* part_l, uint16_t* out,
                 float* out_max, float* out_sum, int tokens, int H, int nsplit, hipStream_t stream) {
    const int64_t grid = (int64_t)tokens * ((H + 1) / 2);
    hipLaunchKernelGGL(merge_kernel, dim3((unsigned)grid), dim3(256), 0, stream, part_o, part_m, part_l, out,
                       out_max, out_sum, H, nsplit);
    return (int)hipGetLastError();
}

}  // namespace dsa
