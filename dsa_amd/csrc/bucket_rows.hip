// Row bucketing of the top-k indices before a prefill-sized forward call (no
// reference counterpart: the reference visits the slots in the order the
// caller gives, dsa/workspace.py:76-141).
//
// out[t, :] is idx[t, :] stably partitioned by kv row range: bucket
// b(x) = x >> shift for a row index 0 <= x < L (shift the least with
// (L - 1) >> shift < 64, so at most 64 buckets of 2^shift rows each), and
// bucket 64 for any other entry (-1 or out of range: a masked slot), in
// bucket order and, within a bucket, in the caller's order.  Attention over
// a token's slots does not depend on their order (a masked slot contributes
// nothing, a duplicate counts twice wherever it sits), so a call on the
// bucketed rows computes the same attention up to the order of its FP32
// sums, and the partition is a fixed function of the row, so repeated calls
// agree bit for bit.  What the order changes is locality: the column-split
// and ping-pong kernels gather a token's rows one 64-slot tile at a time,
// and with every token's tile t drawn from the same row range, workgroups
// that run together on an XCD fetch the same kv rows, which that XCD's L2
// then serves (a full sort gains no more: the order inside a tile does not
// change which rows it fetches).
//
// One workgroup of four waves per token.  Wave w takes the 64-slot chunks
// c = w, w + 4, ...; in each, the lanes of one bucket find each other with
// seven ballots (one per bucket bit), a lane's rank among them is the number
// of such lanes below it, and the lowest writes the chunk's count for the
// bucket.  A scan over chunks then over buckets gives every slot its place,
// (bucket, chunk, rank); the row is assembled in LDS and written coalesced.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace dsa {
namespace {

constexpr int kThreads = 256;
constexpr int kBuckets = 65;  // 64 row ranges + the masked slots

__device__ inline uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// NR: 64-slot chunks per wave (chunks = ceil(topk / 64) <= 4 * NR).
template <int NR>
__global__ __launch_bounds__(kThreads) void bucket_rows_kernel(const int32_t* __restrict__ idx,
                                                               int32_t* __restrict__ out, int topk, uint32_t kv_len,
                                                               int shift) {
    // LDS: counts[chunk][bucket] (then each bucket's offsets within it), the
    // buckets' bases, the assembled row
    extern __shared__ int32_t lds[];
    const int chunks = (topk + 63) >> 6;
    int32_t* counts = lds;
    int32_t* base = lds + chunks * kBuckets;
    int32_t* row_out = base + kBuckets;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const int32_t* src = idx + row * topk;

    // Every load first (clamped into the row; the excess lanes are inactive)
    int32_t val[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) val[r] = src[min(((wave + 4 * r) << 6) + lane, topk - 1)];
    for (int i = tid; i < chunks * kBuckets; i += kThreads) counts[i] = 0;
    __syncthreads();

    // Each slot's bucket and its rank among the chunk's slots of that bucket
    int bucket[NR], rank[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int e = ((wave + 4 * r) << 6) + lane;
        const bool active = e < topk;
        const int b = (uint32_t)val[r] < kv_len ? (int)((uint32_t)val[r] >> shift) : kBuckets - 1;
        // 127 is no bucket: a lane past the row matches no active lane
        const int key = active ? b : 127;
        // This lane's peers (itself included) are the lanes whose key differs
        // in no bit: per bit, the ballot of the bit XOR this lane's bit (0 or
        // ~0), OR-ed into d with one three-input bitwise instruction per half
        // (table 0xDE: d | (m ^ t); the last bit 0x21, its complement, so that
        // d ends as the peers; both symmetric in the outer operands).  Four
        // VALU instructions per bit, against ten for the select-and-AND form.
        uint32_t plo = 0, phi = 0;
        auto key_bit = [&](int bit, uint32_t& t) -> uint64_t {
            t = (uint32_t)__builtin_amdgcn_sbfe(key, bit, 1);
            asm volatile("" : "+v"(t));  // the ballot compares t itself (not a second shift of key)
            return ballot(t != 0);
        };
#pragma unroll
        for (int bit = 0; bit < 6; ++bit) {
            uint32_t t;
            const uint64_t m = key_bit(bit, t);
            plo = __builtin_amdgcn_bitop3_b32((uint32_t)m, plo, t, 0xDE);
            phi = __builtin_amdgcn_bitop3_b32((uint32_t)(m >> 32), phi, t, 0xDE);
        }
        {
            uint32_t t;
            const uint64_t m = key_bit(6, t);
            plo = __builtin_amdgcn_bitop3_b32((uint32_t)m, plo, t, 0x21);
            phi = __builtin_amdgcn_bitop3_b32((uint32_t)(m >> 32), phi, t, 0x21);
        }
        const int below = (int)__builtin_amdgcn_mbcnt_hi(phi, __builtin_amdgcn_mbcnt_lo(plo, 0u));
        if (active && below == 0) counts[(wave + 4 * r) * kBuckets + b] = __popc(plo) + __popc(phi);
        bucket[r] = b;
        rank[r] = below;
    }
    __syncthreads();

    // Per bucket, the exclusive scan over chunks (in place) and the total;
    // wave 0 then scans the totals of buckets 0-63 and wave 1 lane 0 takes
    // the masked bucket, which follows all of them.
    if (tid < kBuckets) {
        int n[4 * NR];
#pragma unroll
        for (int c = 0; c < 4 * NR; ++c) n[c] = c < chunks ? counts[c * kBuckets + tid] : 0;
        int run = 0;
#pragma unroll
        for (int c = 0; c < 4 * NR; ++c) {
            if (c < chunks) counts[c * kBuckets + tid] = run;
            run += n[c];
        }
        if (wave == 0) {
            int incl = run;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int up = __shfl_up(incl, d, 64);
                if (lane >= d) incl += up;
            }
            base[tid] = incl - run;
            if (lane == 63) base[kBuckets - 1] = incl;
        }
    }
    __syncthreads();

#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int c = wave + 4 * r;
        if ((c << 6) + lane < topk) row_out[base[bucket[r]] + counts[c * kBuckets + bucket[r]] + rank[r]] = val[r];
    }
    __syncthreads();
    int32_t* dst = out + row * topk;
    for (int i = tid; i < topk; i += kThreads) dst[i] = row_out[i];
}

}  // namespace

int bucket_shift(int kv_len) {
    int shift = 0;
    while (((uint32_t)(kv_len - 1) >> shift) >= 64u) ++shift;
    return shift;
}

size_t bucket_rows_lds_bytes(int topk) {
    return sizeof(int32_t) * ((size_t)((topk + 63) / 64) * kBuckets + kBuckets + topk);
}

int launch_bucket_rows(const int32_t* idx, int32_t* out, int64_t tokens, int topk, int kv_len, hipStream_t stream) {
    const dim3 grid((unsigned)tokens), block(kThreads);
    const size_t lds = bucket_rows_lds_bytes(topk);
    const uint32_t len = (uint32_t)kv_len;
    const int shift = bucket_shift(kv_len);
    if (topk <= 256)
        hipLaunchKernelGGL(bucket_rows_kernel<1>, grid, block, lds, stream, idx, out, topk, len, shift);
    else if (topk <= 512)
        hipLaunchKernelGGL(bucket_rows_kernel<2>, grid, block, lds, stream, idx, out, topk, len, shift);
    else if (topk <= 1024)
        hipLaunchKernelGGL(bucket_rows_kernel<4>, grid, block, lds, stream, idx, out, topk, len, shift);
    else if (topk <= 2048)
        hipLaunchKernelGGL(bucket_rows_kernel<8>, grid, block, lds, stream, idx, out, topk, len, shift);
    else
        hipLaunchKernelGGL(bucket_rows_kernel<16>, grid, block, lds, stream, idx, out, topk, len, shift);
    return (int)hipGetLastError();
}

}  // namespace dsa
