// Lightning indexer for gfx950 (MI355X): the token selector that produces
// the `indices` the sparse attention consumes.  No counterpart in the
// reference, which takes the indices as an input (README.md:19-21).
//
//   logits[t, s] = sum_j w[t, j] * relu(q[t, j, :] . k[s, :])      s < len[t]
//   indices[t]   = the TOPK keys s < len[t] of largest logit (ties: lower s
//                  first), in ascending s order, padded with -1
//
// q [B, SQ, HI, 128] bf16 (HI = 32 or 64), k [B, L, 128] bf16 (one key per
// token, shared by the heads), w [B, SQ, HI] fp32, len [B, SQ] int32.
//
// Logits kernel: one workgroup owns 256 / HI queries of one batch (256 query
// heads) and a range of 64-key tiles.  Keys stream through a two-stage LDS
// ring (buffer_load ... lds, 16 KiB per tile, 16-byte chunks XOR-swizzled by
// row); every wave holds the Q fragments of 64 query heads in VGPRs and
// computes C[head, key] with v_mfma_f32_32x32x16_bf16 (A = Q, B = K^T from
// LDS), then the ReLU and the weighted sum over heads in registers: each lane
// holds 16 heads of one key, its partner lane (l ^ 32) the other 16.
//
// Top-k kernel: one 1024-thread workgroup per query row.  A 4-pass radix
// select (8 bits per pass, LDS histograms) over order-preserving 32-bit keys
// of the logits finds the TOPK-th largest key T; a compaction pass then keeps
// every s with key > T and the lowest-s ties == T, writing them in ascending
// order with block-wide prefix counts.  Rows of up to 32768 candidates are
// cached in LDS after the first read.
#include <hip/hip_runtime.h>
#include <float.h>
#include <stdint.h>

#include "kernels.h"

namespace dsa {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef int rsrc_t __attribute__((ext_vector_type(4)));

constexpr int kDim = 128;                         // indexer head dimension
constexpr int kKeyTile = 64;                      // keys per ring stage
constexpr int kTileBytes = kKeyTile * kDim * 2;   // 16 KiB
constexpr int kLoadsPerWave = kTileBytes / 1024 / 4;  // 1 KiB per instruction, 4 waves

template <typename T>
__device__ __forceinline__ T lds_load(uint32_t addr) {
    return *reinterpret_cast<__attribute__((address_space(3))) T*>(addr);
}
template <typename T>
__device__ __forceinline__ void lds_store(uint32_t addr, T v) {
    *reinterpret_cast<__attribute__((address_space(3))) T*>(addr) = v;
}

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    rsrc_t r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff));
    r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
    r[3] = 0x00020000;
    return r;
}

// Sum over lanes l and l ^ 32 (v_permlane32_swap on two copies of v).
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One 1 KiB slice of a key tile (4 key rows x 256 B) straight into LDS: lane
// l lands at m0 + 16 l, i.e. row l / 16, physical chunk l % 16, and loads the
// logical chunk (l % 16) ^ (row % 16) of that row, so the B-fragment reads
// below (16 rows x the same logical chunk per quarter-wave) hit 64 distinct
// banks.  Rows past L read zeros: the whole offset is in the VGPR operand,
// which the buffer range check covers (the SGPR offset is not checked).
__device__ __forceinline__ void load_slice(uint32_t lds_dst, rsrc_t rsrc, uint32_t tile_off, int slice, int lane) {
    const int row = slice * 4 + (lane >> 4);
    const uint32_t voff = tile_off + (uint32_t)row * 256u + ((uint32_t)((lane & 15) ^ (row & 15)) << 4);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(__builtin_amdgcn_readfirstlane(lds_dst)), "v"(voff), "s"(rsrc)
        : "memory", "m0");
#pragma clang diagnostic pop
}

template <int HI>
__global__ __launch_bounds__(256, 1) void indexer_logits_kernel(IndexerParams p) {
    static_assert(HI == 32 || HI == 64, "indexer heads");
    constexpr int TG = 256 / HI;  // queries per workgroup
    __shared__ __attribute__((aligned(1024))) char smem[2 * kTileBytes];
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int b = blockIdx.x / p.tgroups;
    const int t0 = (blockIdx.x % p.tgroups) * TG;

    // Key tiles of this workgroup, cut at the longest candidate range of its queries.
    int maxlen = 0;
#pragma unroll
    for (int i = 0; i < TG; ++i)
        if (t0 + i < p.SQ) maxlen = max(maxlen, min(max(p.len[(int64_t)b * p.SQ + t0 + i], 0), p.L));
    const int tile_begin = blockIdx.y * p.tiles_per_wg;
    const int tile_end = min(min(tile_begin + p.tiles_per_wg, p.ntiles), (maxlen + kKeyTile - 1) / kKeyTile);
    if (tile_begin >= tile_end) return;  // uniform: the whole workgroup leaves

    // This wave's two 32-head blocks: rows (2 * wave + hb) * 32 .. + 31 of the
    // workgroup's TG * HI query heads.  A fragments (lane: head rowbase + l % 32,
    // dims 16 ks + 8 (l / 32) .. + 7) and the weights of the 16 heads whose
    // products this lane accumulates (C row 8 (r / 4) + 4 (l / 32) + r % 4).
    bf16x8 qa[2][8];
    float wv[2][16];
    int tok[2], qlen[2];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
        const int rowbase = (2 * wave + hb) * 32;
        const int t = t0 + rowbase / HI;
        tok[hb] = t;
        const bool live = t < p.SQ;
        const int64_t qt = (int64_t)b * p.SQ + (live ? t : 0);
        qlen[hb] = live ? min(max(p.len[qt], 0), p.L) : 0;
        const uint16_t* qrow = p.q + (qt * HI + rowbase % HI + (lane & 31)) * kDim + 8 * (lane >> 5);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) qa[hb][ks] = *reinterpret_cast<const bf16x8*>(qrow + 16 * ks);
        const float* wrow = p.w + qt * HI + rowbase % HI;
#pragma unroll
        for (int r = 0; r < 16; ++r) wv[hb][r] = live ? wrow[8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)] : 0.f;
    }

    const rsrc_t kr = make_rsrc(p.k + (int64_t)b * p.L * kDim, (uint32_t)p.L * kDim * 2u);
    auto issue = [&](int tile) {
        const uint32_t dst = lds + (uint32_t)(tile & 1) * kTileBytes;
#pragma unroll
        for (int i = 0; i < kLoadsPerWave; ++i) {
            const int slice = wave * kLoadsPerWave + i;
            load_slice(dst + slice * 1024, kr, (uint32_t)tile * kTileBytes, slice, lane);
        }
    };

    issue(tile_begin);
    wait_vmcnt<0>();  // Q, weights and the first tile: nothing the compiler waits for stays in the loop

    float res[2][2];  // [hb][key block] sums of the previous tile, stored one iteration late
    int prev = -1;
    for (int tile = tile_begin; tile < tile_end; ++tile) {
        wait_vmcnt<0>();  // this tile (and last iteration's stores, issued before it)
        lds_barrier();    // tile visible; every wave is past the previous tile's reads
        // Stores of the previous tile, then the next tile's loads (so the wait
        // above never drains a load issued after a store).
        if (prev >= 0) {
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                if constexpr (HI == 64)
                    if (hb == 1) break;  // both blocks belong to one query: summed into res[0]
                const int t = tok[hb];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const int s = prev * kKeyTile + kb * 32 + (lane & 31);
                    if (lane < 32 && t < p.SQ && s < p.L)
                        p.logits[((int64_t)b * p.SQ + t) * p.L + s] = s < qlen[hb] ? res[hb][kb] : -INFINITY;
                }
            }
        }
        if (tile + 1 < tile_end) issue(tile + 1);

        const uint32_t stage = lds + (uint32_t)(tile & 1) * kTileBytes;
        f32x16 acc[2][2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) acc[hb][kb] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                // B fragment: key row kb * 32 + l % 32, logical chunk 2 ks + l / 32.
                const int row = kb * 32 + (lane & 31);
                const bf16x8 bk = lds_load<bf16x8>(stage + row * 256 + (((2 * ks + (lane >> 5)) ^ (row & 15)) << 4));
#pragma unroll
                for (int hb = 0; hb < 2; ++hb)
                    acc[hb][kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[hb][ks], bk, acc[hb][kb], 0, 0, 0);
            }
        }
        // ReLU, weights, sum over this lane's 16 heads, then over the partner lane's 16.
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                float sum = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) sum = fmaf(wv[hb][r], fmaxf(acc[hb][kb][r], 0.f), sum);
                res[hb][kb] = sum_xor32(sum);
            }
        if constexpr (HI == 64) {  // the query's 64 heads are this wave's two blocks
            res[0][0] += res[1][0];
            res[0][1] += res[1][1];
        }
        prev = tile;
    }
    // Last tile's stores.
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
        if constexpr (HI == 64)
            if (hb == 1) break;
        const int t = tok[hb];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int s = prev * kKeyTile + kb * 32 + (lane & 31);
            if (lane < 32 && t < p.SQ && s < p.L)
                p.logits[((int64_t)b * p.SQ + t) * p.L + s] = s < qlen[hb] ? res[hb][kb] : -INFINITY;
        }
    }
}

// ------------------------------------------------------------------ top-k
constexpr int kTopkThreads = 1024;
constexpr int kCacheKeys = 32768;  // candidates kept in LDS (128 KiB)

// Order-preserving map of a float to an unsigned key (larger float, larger key).
__device__ __forceinline__ uint32_t float_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(kTopkThreads, 1) void indexer_topk_kernel(const float* __restrict__ logits,
                                                                      const int32_t* __restrict__ len,
                                                                      int32_t* __restrict__ out, int L, int K) {
    __shared__ uint32_t cache[kCacheKeys];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t wave_cnt[2][kTopkThreads / 64];
    __shared__ uint32_t shared_word[4];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = min(max(len[row], 0), L);
    const float* src = logits + (int64_t)row * L;
    int32_t* dst = out + (int64_t)row * K;

    if (n <= K) {  // every candidate is selected
        for (int j = tid; j < K; j += kTopkThreads) dst[j] = j < n ? j : -1;
        return;
    }
    const bool cached = n <= kCacheKeys;
    auto key_at = [&](int s) -> uint32_t { return cached ? cache[s] : float_key(src[s]); };

    uint32_t prefix = 0, mask = 0;
    int remaining = K;  // keys still to take among those matching prefix under mask
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < 256; i += kTopkThreads) hist[i] = 0;
        __syncthreads();
        for (int s = tid; s < n; s += kTopkThreads) {
            uint32_t u;
            if (pass == 0) {
                u = float_key(src[s]);
                if (cached) cache[s] = u;
            } else {
                u = key_at(s);
            }
            if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            // Suffix counts over the 256 bins, four bins per lane from the top.
            uint32_t c[4], sum = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = hist[255 - (4 * lane + j)];
                sum += c[j];
            }
            // inclusive scan of the per-lane sums across the wave (bins from the top)
            uint32_t incl = sum;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t o = __shfl_up(incl, d);
                if (lane >= d) incl += o;
            }
            uint32_t above = incl - sum;  // keys in bins above this lane's four
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (above < (uint32_t)remaining && above + c[j] >= (uint32_t)remaining) {
                    shared_word[0] = 255 - (4 * lane + j);  // the bin holding the remaining-th key
                    shared_word[1] = above;
                }
                above += c[j];
            }
        }
        __syncthreads();
        const uint32_t digit = shared_word[0];
        remaining -= (int)shared_word[1];
        prefix |= digit << shift;
        mask |= 255u << shift;
        __syncthreads();  // shared_word is rewritten by the next pass
    }
    // Threshold key T = prefix; `remaining` ties (key == T) are taken, lowest s first.
    const uint32_t thr = prefix;
    uint32_t taken = 0, ties = 0;  // running totals over the chunks before this one
#pragma unroll 1
    for (int base = 0; base < n; base += kTopkThreads) {
        const int s = base + tid;
        const uint32_t u = s < n ? key_at(s) : 0u;
        const bool tie = s < n && u == thr;
        const uint64_t tie_mask = __ballot(tie);
        const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        const uint32_t tie_rank_wave = (uint32_t)__popcll(tie_mask & below);
        if (lane == 0) wave_cnt[0][wave] = (uint32_t)__popcll(tie_mask);
        __syncthreads();
        uint32_t tie_before = ties;
        for (int w = 0; w < wave; ++w) tie_before += wave_cnt[0][w];
        const bool sel = s < n && (u > thr || (tie && tie_before + tie_rank_wave < (uint32_t)remaining));
        const uint64_t sel_mask = __ballot(sel);
        if (lane == 0) wave_cnt[1][wave] = (uint32_t)__popcll(sel_mask);
        __syncthreads();
        uint32_t pos = taken + (uint32_t)__popcll(sel_mask & below);
        uint32_t chunk_sel = 0, chunk_tie = 0;
        for (int w = 0; w < kTopkThreads / 64; ++w) {
            if (w < wave) pos += wave_cnt[1][w];
            chunk_sel += wave_cnt[1][w];
            chunk_tie += wave_cnt[0][w];
        }
        if (sel && pos < (uint32_t)K) dst[pos] = s;
        taken += chunk_sel;
        ties += chunk_tie;
        __syncthreads();  // wave_cnt is rewritten by the next chunk
    }
}

}  // namespace

int launch_indexer_logits(const IndexerParams& p, hipStream_t stream) {
    const dim3 grid((unsigned)(p.B * p.tgroups), (unsigned)((p.ntiles + p.tiles_per_wg - 1) / p.tiles_per_wg));
    if (p.HI == 64)
        hipLaunchKernelGGL(indexer_logits_kernel<64>, grid, dim3(256), 0, stream, p);
    else if (p.HI == 32)
        hipLaunchKernelGGL(indexer_logits_kernel<32>, grid, dim3(256), 0, stream, p);
    else
        return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

int launch_indexer_topk(const float* logits, const int32_t* len, int32_t* indices, int rows, int L, int topk,
                        hipStream_t stream) {
    hipLaunchKernelGGL(indexer_topk_kernel, dim3((unsigned)rows), dim3(kTopkThreads), 0, stream, logits, len,
                       indices, L, topk);
    return (int)hipGetLastError();
}

}  // namespace dsa
