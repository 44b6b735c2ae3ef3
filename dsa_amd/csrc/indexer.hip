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
// Logits kernel: one workgroup owns 256 / HI / KS queries of one batch and a
// range of key stages of KS x 64 keys.  Keys stream through a two-stage LDS
// ring (buffer_load ... lds, 16 KiB per 64 keys, 16-byte chunks XOR-swizzled
// by row); every wave holds the Q fragments of 64 query heads in VGPRs and
// computes C[head, key] for one 64-key sub-tile of the stage with
// v_mfma_f32_32x32x16_bf16 (A = Q, B = K^T from LDS), then the ReLU and the
// weighted sum over heads in registers: each lane holds 16 heads of one key,
// its partner lane (l ^ 32) the other 16.  KS (1, 2, 4) is the number of
// waves sharing a query: 4 for single-query decode, 1 for prefill.
//
// Top-k kernel: one 1024-thread workgroup per query row.  A radix select over
// order-preserving 32-bit keys of the logits finds the TOPK-th largest key T:
// a 12-bit first digit over every candidate (4096 LDS bins, wide enough that
// the atomics of clustered logits rarely collide), a 4-bit digit over the
// LDS-cached upper halves of the keys, then two 8-bit digits over the few
// entries that share T's upper 16 bits, gathered into LDS.  One sweep keeps
// every s with key > T and the lowest-s ties == T, written in ascending
// order.  A row of up to 65536 candidates is read from memory once, plus its
// gathered entries.
#include <hip/hip_runtime.h>
#include <type_traits>
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

// KS wave groups split every key stage (KS x 64 keys) and the workgroup's
// 4 / KS query slots (64 query heads each) share it: KS = 1 for prefill (4
// slots reuse each key tile), 2 or 4 when SQ is too small to fill the slots.
template <int HI, int KS>
__global__ __launch_bounds__(256, 1) void indexer_logits_kernel(IndexerParams p) {
    static_assert(HI == 32 || HI == 64, "indexer heads");
    static_assert(KS == 1 || KS == 2 || KS == 4, "key split");
    constexpr int TG = 256 / HI / KS;            // queries per workgroup
    constexpr int kStageBytes = KS * kTileBytes;  // one ring stage: KS x 64 keys
    __shared__ __attribute__((aligned(1024))) char smem[2 * kStageBytes];
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qg = wave / KS;  // this wave's query slot
    const int kg = wave % KS;  // this wave's 64-key sub-tile of every stage
    const int b = blockIdx.x / p.tgroups;
    const int t0 = (blockIdx.x % p.tgroups) * TG;

    // Key stages of this workgroup, cut at the longest candidate range of its queries.
    int maxlen = 0;
#pragma unroll
    for (int i = 0; i < TG; ++i)
        if (t0 + i < p.SQ) maxlen = max(maxlen, min(max(p.len[(int64_t)b * p.SQ + t0 + i], 0), p.L));
    const int tile_begin = blockIdx.y * p.tiles_per_wg;
    const int tile_end =
        min(min(tile_begin + p.tiles_per_wg, p.ntiles), (maxlen + kKeyTile * KS - 1) / (kKeyTile * KS));
    if (tile_begin >= tile_end) return;  // uniform: the whole workgroup leaves

    // This wave's two 32-head blocks: rows (2 * qg + hb) * 32 .. + 31 of the
    // workgroup's TG * HI query heads.  A fragments (lane: head rowbase + l % 32,
    // dims 16 ks + 8 (l / 32) .. + 7) and the weights of the 16 heads whose
    // products this lane accumulates (C row 8 (r / 4) + 4 (l / 32) + r % 4).
    bf16x8 qa[2][8];
    float wv[2][16];
    int tok[2], qlen[2];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
        const int rowbase = (2 * qg + hb) * 32;
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
        const uint32_t dst = lds + (uint32_t)(tile & 1) * kStageBytes;
#pragma unroll
        for (int i = 0; i < kLoadsPerWave * KS; ++i) {
            const int slice = wave * kLoadsPerWave * KS + i;
            load_slice(dst + slice * 1024, kr, (uint32_t)tile * kStageBytes, slice, lane);
        }
    };
    auto store = [&](int tile, const float (&res)[2][2]) {
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            if constexpr (HI == 64)
                if (hb == 1) break;  // both blocks belong to one query: summed into res[0]
            const int t = tok[hb];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int s = (tile * KS + kg) * kKeyTile + kb * 32 + (lane & 31);
                if (lane < 32 && t < p.SQ && s < p.L)
                    p.logits[((int64_t)b * p.SQ + t) * p.L + s] = s < qlen[hb] ? res[hb][kb] : -INFINITY;
            }
        }
    };

    issue(tile_begin);
    wait_vmcnt<0>();  // Q, weights and the first stage: nothing the compiler waits for stays in the loop

    float res[2][2];  // [hb][key block] sums of the previous stage, stored one iteration late
    int prev = -1;
    for (int tile = tile_begin; tile < tile_end; ++tile) {
        wait_vmcnt<0>();  // this stage (and last iteration's stores, issued before it)
        lds_barrier();    // stage visible; every wave is past the previous stage's reads
        // Stores of the previous stage, then the next stage's loads (so the wait
        // above never drains a load issued after a store).
        if (prev >= 0) store(prev, res);
        if (tile + 1 < tile_end) issue(tile + 1);

        const uint32_t stage = lds + (uint32_t)(tile & 1) * kStageBytes + (uint32_t)kg * kTileBytes;
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
    store(prev, res);  // last stage
}

// ------------------------------------------------------------------ top-k
constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;
constexpr int kChunk = 256;        // entries one wave covers per step: 4 consecutive per lane
constexpr int kCacheKeys = 65536;  // bits 31..16 of every candidate's key cached in LDS (128 KiB)
constexpr int kBins0 = 4096;       // first digit: key bits 31..20 (sign, exponent, 3 mantissa bits)
constexpr int kCandCap = 1536;     // entries sharing T's upper 16 bits kept in LDS as (s, key)

struct TopkShared {
    __attribute__((aligned(16))) uint16_t hi16[kCacheKeys];
    uint32_t hist[kBins0];  // digit histograms; afterwards 2 flag bits per cached s
    uint32_t cand_s[kCandCap];
    uint32_t cand_key[kCandCap];
    uint32_t wgt[kTopkWaves];  // per wave segment: entries with key > T
    uint32_t weq[kTopkWaves];  // per wave segment: entries with key == T
    uint32_t word[4];
};

// Order-preserving map of a float to an unsigned key (larger float, larger key).
__device__ __forceinline__ uint32_t float_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t lanes_below(int lane) { return lane == 0 ? 0ull : (~0ull >> (64 - lane)); }

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
    return v;
}

// Inclusive prefix sum across the wave (lane order).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(v, d);
        if (lane >= d) v += o;
    }
    return v;
}

// One row of logits behind a range-checked buffer descriptor: reads at or past
// n return 0.0 (so the caller masks them), and being intrinsics the loads are
// never wrapped in per-lane branches.
struct Row {
    __amdgpu_buffer_rsrc_t rs;
    __device__ __forceinline__ uint32_t key(int s) const {
        return float_key(__uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, s * 4, 0, 0)));
    }
};

// Rank of this lane among the lanes whose bit is set in m (lanes below it).
__device__ __forceinline__ uint32_t lane_rank(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Exclusive prefix over the lanes, and wave total, of a per-lane count c in
// [0, 7]: one ballot per bit of c.
__device__ __forceinline__ void lane_prefix3(uint32_t c, uint32_t& before, uint32_t& total) {
    before = 0;
    total = 0;
#pragma unroll
    for (int b = 0; b < 3; ++b) {
        const uint64_t m = __ballot((c >> b) & 1u);
        before += lane_rank(m) << b;
        total += (uint32_t)__popcll(m) << b;
    }
}

// 4-bit masks over entries j = 0..3: h[j] > x, h[j] == x.
__device__ __forceinline__ uint32_t mask_gt4(const uint32_t h[4], uint32_t x) {
    return (h[0] > x ? 1u : 0u) | (h[1] > x ? 2u : 0u) | (h[2] > x ? 4u : 0u) | (h[3] > x ? 8u : 0u);
}
__device__ __forceinline__ uint32_t mask_eq4(const uint32_t h[4], uint32_t x) {
    return (h[0] == x ? 1u : 0u) | (h[1] == x ? 2u : 0u) | (h[2] == x ? 4u : 0u) | (h[3] == x ? 8u : 0u);
}

// Entries s .. s + 3 below hi, as a 4-bit mask.
__device__ __forceinline__ uint32_t valid4(int s, int hi) {
    const int left = hi - s;
    return left >= 4 ? 15u : (left <= 0 ? 0u : (1u << left) - 1u);
}

// Upper key halves of entries s .. s + 3 of one wave step (s = base + 4 lane,
// base a multiple of kChunk below hi): from the LDS cache, or from memory.
template <bool CACHED>
__device__ __forceinline__ void upper4(const TopkShared& sh, const Row& row, int base, int s, uint32_t h[4]) {
    if constexpr (CACHED) {
        (void)base;
        const uint2 v = *reinterpret_cast<const uint2*>(&sh.hi16[s]);
        h[0] = v.x & 0xffffu;
        h[1] = v.x >> 16;
        h[2] = v.y & 0xffffu;
        h[3] = v.y >> 16;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = row.key(s + j) >> 16;
    }
}

// Per row: the threshold key T (the K-th largest key) and the number of
// entries equal to T to take, found digit by digit, then one sweep that
// writes the selected s in ascending order.  Each wave owns a contiguous
// segment of s, walked kChunk entries at a time.
//   digit 0, bits 31..20: one read of the row; caches the keys' bits 31..16
//   digit 1, bits 19..16: entries of digit 0's bin, from the cache; also
//           counts per segment the entries whose upper 16 bits exceed T's
//   gather: the entries sharing T's upper 16 bits (typically a few hundred)
//           as (s, key) into LDS -- one batch of independent loads
//   digits 2, 3, bits 15..8 and 7..0: over the gathered entries, which then
//           get flags (key > T, key == T) and per-segment counts
//   sweep: the segment counts place every wave's writes.
// CACHED = false (rows longer than the cache) reads the row from memory in
// every pass; a 16-bit prefix shared by more than kCandCap entries is
// resolved over the whole row, reading keys from memory.
template <bool CACHED>
__device__ __forceinline__ void topk_select(TopkShared& sh, const Row& row, int32_t* __restrict__ dst, int n,
                                            int K) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: segment bounds live in SGPRs
    const int seg = (n + kTopkWaves * kChunk - 1) / (kTopkWaves * kChunk) * kChunk;
    const int lo = min(wave * seg, n), hi = min(lo + seg, n);  // this wave's entries [lo, hi)
    constexpr int U = 4;  // wave steps per loop iteration (loads in flight)

    // ---- digit 0 (bits 31..20) over every candidate; caches bits 31..16
    for (int i = tid; i < kBins0; i += kTopkThreads) sh.hist[i] = 0;
    if (tid < kTopkWaves) sh.weq[tid] = 0;
    if (tid == 0) sh.word[2] = 0;
    __syncthreads();
    for (int base = lo; base < hi; base += 2 * U * kChunk) {
        // lane-interleaved: entry base + c * 64 + lane, every load 256 contiguous bytes
        uint32_t k[2 * U * 4];
#pragma unroll
        for (int c = 0; c < 2 * U * 4; ++c) k[c] = row.key(base + c * 64 + lane);
#pragma unroll
        for (int c = 0; c < 2 * U * 4; ++c) {
            const int s = base + c * 64 + lane;
            if constexpr (CACHED)
                if (base + (c / 4) * kChunk < hi) sh.hi16[s] = (uint16_t)(k[c] >> 16);  // step inside the cache
            if (s < hi) atomicAdd(&sh.hist[k[c] >> 20], 1u);
        }
    }
    __syncthreads();
    uint32_t need = (uint32_t)K;  // entries still to take among those matching the digits so far
    {
        // thread tid owns bins kBins0 - 1 - 4 tid - j (j = 0..3), counted from the top
        uint32_t c[4], mine = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            c[j] = sh.hist[kBins0 - 1 - 4 * tid - j];
            mine += c[j];
        }
        const uint32_t incl = wave_incl_scan(mine, lane);
        if (lane == 63) sh.wgt[wave] = incl;
        __syncthreads();
        uint32_t above = incl - mine;
        for (int w = 0; w < wave; ++w) above += sh.wgt[w];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (above < need && above + c[j] >= need) {  // exactly one (thread, j) crosses
                sh.word[0] = (uint32_t)(kBins0 - 1 - 4 * tid - j);
                sh.word[1] = above;
            }
            above += c[j];
        }
        __syncthreads();
    }
    const uint32_t bin0 = sh.word[0];
    need -= sh.word[1];
    __syncthreads();  // hist, word and wgt are rewritten below

    // ---- digit 1 (bits 19..16): per-wave 16-bin histograms of digit 0's bin
    if (tid < kTopkWaves * 16) sh.hist[tid] = 0;
    __syncthreads();
    {
        uint32_t above0 = 0;  // entries of this segment in bins above bin0
        for (int base = lo; base < hi; base += U * kChunk) {
            uint32_t h[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (base + u * kChunk < hi) {
                    upper4<CACHED>(sh, row, base + u * kChunk, base + u * kChunk + 4 * lane, h[u]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) h[u][j] = 0;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int s = base + u * kChunk + 4 * lane;
                const uint32_t vm = valid4(s, hi);
                // bins above bin0: upper halves >= (bin0 + 1) << 4
                above0 += (uint32_t)__popc(mask_gt4(h[u], (bin0 << 4) | 15u) & vm);
                uint32_t d0[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) d0[j] = h[u][j] >> 4;
                const uint32_t inb = mask_eq4(d0, bin0) & vm;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if ((inb >> j) & 1u) atomicAdd(&sh.hist[wave * 16 + (h[u][j] & 15u)], 1u);
            }
        }
        above0 = wave_sum(above0);
        if (lane == 0) sh.wgt[wave] = above0;
    }
    __syncthreads();
    if (wave == 0) {  // lane l < 16 holds bin 15 - l
        uint32_t c = 0;
        if (lane < 16)
            for (int w = 0; w < kTopkWaves; ++w) c += sh.hist[w * 16 + 15 - lane];
        const uint32_t above = wave_incl_scan(c, lane) - c;
        if (lane < 16 && above < need && above + c >= need) {
            sh.word[0] = 15 - lane;
            sh.word[1] = above;
            sh.word[3] = c;
        }
    }
    __syncthreads();
    const uint32_t digit1 = sh.word[0];
    const uint32_t pre16 = (bin0 << 4) | digit1;
    const uint32_t in16 = sh.word[3];
    need -= sh.word[1];
    if (tid < kTopkWaves) {  // segment counts of entries whose upper 16 bits exceed pre16
        uint32_t c = sh.wgt[tid];
        for (uint32_t d = digit1 + 1; d < 16; ++d) c += sh.hist[tid * 16 + d];
        sh.wgt[tid] = c;
    }
    __syncthreads();

    // ---- gather the entries sharing the 16-bit prefix (when they fit)
    const bool gathered = in16 <= (uint32_t)kCandCap;
    if (gathered) {
        for (int base = lo; base < hi; base += U * kChunk) {
            uint32_t h[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (base + u * kChunk < hi) {
                    upper4<CACHED>(sh, row, base + u * kChunk, base + u * kChunk + 4 * lane, h[u]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) h[u][j] = 0;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int s = base + u * kChunk + 4 * lane;
                const uint32_t hit = mask_eq4(h[u], pre16) & valid4(s, hi);
                if (__ballot(hit != 0u)) {  // wave-uniform
                    uint32_t off, total;
                    lane_prefix3((uint32_t)__popc(hit), off, total);
                    uint32_t at = 0;
                    if (lane == 0) at = atomicAdd(&sh.word[2], total);
                    at = (uint32_t)__builtin_amdgcn_readfirstlane((int)at) + off;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if ((hit >> j) & 1u) sh.cand_s[at++] = (uint32_t)(s + j);
                }
            }
        }
        __syncthreads();
        for (int i = tid; i < (int)in16; i += kTopkThreads) sh.cand_key[i] = row.key((int)sh.cand_s[i]);
        __syncthreads();
    }

    // ---- digits 2, 3 (bits 15..8, 7..0) over the gathered entries (else over the row)
    uint32_t prefix = pre16 << 16, mask = 0xffff0000u;
#pragma unroll 1
    for (int shift = 8; shift >= 0; shift -= 8) {
        if (tid < 256) sh.hist[tid] = 0;
        __syncthreads();
        if (gathered) {
            for (int i = tid; i < (int)in16; i += kTopkThreads) {
                const uint32_t u = sh.cand_key[i];
                if ((u & mask) == prefix) atomicAdd(&sh.hist[(u >> shift) & 255], 1u);
            }
        } else {
            for (int s = tid; s < n; s += kTopkThreads) {
                const uint32_t u = row.key(s);
                if ((u & mask) == prefix) atomicAdd(&sh.hist[(u >> shift) & 255], 1u);
            }
        }
        __syncthreads();
        if (wave == 0) {  // four bins per lane from the top
            uint32_t c[4], sum = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = sh.hist[255 - (4 * lane + j)];
                sum += c[j];
            }
            uint32_t above = wave_incl_scan(sum, lane) - sum;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (above < need && above + c[j] >= need) {
                    sh.word[0] = 255 - (4 * lane + j);
                    sh.word[1] = above;
                }
                above += c[j];
            }
        }
        __syncthreads();
        need -= sh.word[1];
        prefix |= sh.word[0] << shift;
        mask |= 255u << shift;
        __syncthreads();  // word and hist are rewritten next
    }
    const uint32_t thr = prefix;

    // ---- segment counts (and, for a cached row, flags) of the entries sharing pre16
    if (CACHED && gathered)
        for (int i = tid; i < kBins0; i += kTopkThreads) sh.hist[i] = 0;
    __syncthreads();
    if (gathered) {
        for (int i = tid; i < (int)in16; i += kTopkThreads) {
            const uint32_t u = sh.cand_key[i], s = sh.cand_s[i];
            const int w = (int)s / seg;
            if (u > thr) atomicAdd(&sh.wgt[w], 1u);
            if (u == thr) atomicAdd(&sh.weq[w], 1u);
            if constexpr (CACHED) {
                const uint32_t f = (u > thr ? 1u : 0u) | (u == thr ? 2u : 0u);
                if (f) atomicOr(&sh.hist[s >> 4], f << (2 * (s & 15)));
            }
        }
    } else {
        uint32_t ng = 0, ne = 0;
        for (int s = lo + lane; s < hi; s += 64) {
            const uint32_t u = row.key(s);
            ng += ((u >> 16) == pre16 && u > thr) ? 1u : 0u;
            ne += u == thr ? 1u : 0u;
        }
        ng = wave_sum(ng);
        ne = wave_sum(ne);
        if (lane == 0) {
            sh.wgt[wave] += ng;
            sh.weq[wave] = ne;
        }
    }
    __syncthreads();

    // ---- output: every s with key > T, then the first `need` with key == T, ascending s
    uint32_t pos = 0, ties = 0;
    for (int w = 0; w < wave; ++w) {
        pos += sh.wgt[w];
        ties += sh.weq[w];
    }
    pos += min(ties, need);
    const bool flags = CACHED && gathered;
    for (int base = lo; base < hi; base += U * kChunk) {
        uint32_t h[U][4], f8[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            f8[u] = 0;
            if (base + u * kChunk < hi) {
                const int s = base + u * kChunk + 4 * lane;
                upper4<CACHED>(sh, row, base + u * kChunk, s, h[u]);
                // flag bits of entries s .. s + 3: byte (s % 16) / 4 of flag word s / 16
                if (flags) f8[u] = (sh.hist[s >> 4] >> (8 * (lane & 3))) & 0xffu;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) h[u][j] = 0;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = base + u * kChunk + 4 * lane;
            const uint32_t vm = valid4(s, hi);
            const uint32_t mid = mask_eq4(h[u], pre16) & vm;  // share T's upper 16 bits
            const uint32_t f = f8[u];
            // de-interleave the flags: bit 2j = key > T, bit 2j + 1 = key == T
            const uint32_t fgt = (f & 1u) | ((f >> 1) & 2u) | ((f >> 2) & 4u) | ((f >> 3) & 8u);
            const uint32_t feq = ((f >> 1) & 1u) | ((f >> 2) & 2u) | ((f >> 3) & 4u) | ((f >> 4) & 8u);
            uint32_t gtm = (mask_gt4(h[u], pre16) & vm) | (mid & fgt);
            uint32_t eqm = mid & feq;
            if (!flags && __ballot(mid != 0u)) {  // keys of the entries sharing pre16, from memory
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t key = row.key(s + j);
                    const uint32_t bit = mid & (1u << j);
                    gtm |= key > thr ? bit : 0u;
                    eqm |= key == thr ? bit : 0u;
                }
            }
            uint32_t selm = gtm, tie_total = 0;
            if (__ballot(eqm != 0u)) {  // rare: this step holds entries equal to T
                uint32_t tie_off;
                lane_prefix3((uint32_t)__popc(eqm), tie_off, tie_total);
                uint32_t rank = ties + tie_off;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if ((eqm >> j) & 1u) {
                        if (rank < need) selm |= 1u << j;
                        ++rank;
                    }
                }
            }
            uint32_t sel_off, sel_total;
            lane_prefix3((uint32_t)__popc(selm), sel_off, sel_total);
            uint32_t at = pos + sel_off;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if ((selm >> j) & 1u) {
                    if (at < (uint32_t)K) dst[at] = s + j;
                    ++at;
                }
            }
            pos += sel_total;
            ties += tie_total;
        }
    }
}

__global__ __launch_bounds__(kTopkThreads, 1) void indexer_topk_kernel(const float* __restrict__ logits,
                                                                      const int32_t* __restrict__ len,
                                                                      int32_t* __restrict__ out, int L, int K) {
    __shared__ TopkShared sh;
    const int r = blockIdx.x;
    const int n = min(max(len[r], 0), L);
    int32_t* dst = out + (int64_t)r * K;
    if (n <= K) {  // every candidate is selected
        for (int j = threadIdx.x; j < K; j += kTopkThreads) dst[j] = j < n ? j : -1;
        return;
    }
    const Row row{__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(logits + (int64_t)r * L), (short)0, n * 4,
                                                    0x00020000)};
    if (n <= kCacheKeys)
        topk_select<true>(sh, row, dst, n, K);
    else
        topk_select<false>(sh, row, dst, n, K);
}

// ------------------------------------------------ segmented top-k (few rows)
// With few rows, one 1024-thread workgroup per row leaves most CUs idle and is
// bound by its own VALU issue.  The segmented path splits every row over
// kSegWgs workgroups of 256 threads, each owning the contiguous segment
// [p * seg, (p + 1) * seg) of s, in three launches (the kernel boundaries are
// the only synchronisation; the workspace needs no initialisation):
//   1. seg_hist: per segment, the histogram of the keys' bits 31..20;
//   2. seg_cand: every workgroup finds, from its row's histograms, the bin
//      bin0 holding the TOPK-th largest key; it records how many of its
//      entries lie above bin0 and stores the keys of its entries in bin0
//      (the candidates) in its own range of the row's candidate list;
//   3. seg_emit: every workgroup resolves, from the candidates, the threshold
//      key T and how many entries equal to T each segment takes (ties go to
//      the lowest s, i.e. to the earliest segments), then writes its selected
//      s in ascending order at its offset: key > T, or key == T among its
//      first takes.
// Same selection and order as topk_select.
constexpr int kSegWgs = 8;          // workgroups per row
constexpr int kSegThreads = 256;
constexpr int kSegMaxRows = 32;     // rows * kSegWgs workgroups at most: 256
constexpr int kSegCandCap = 8192;   // candidates resolved from LDS; more are read from the workspace
constexpr int kSegKeys = 16;        // keys per thread in flight (4096 per workgroup and batch)

// Workspace words of one row: histograms [kSegWgs][kBins0] of key bits
// 31..20 and coarse ones [kSegWgs][kCoarse] of bits 31..26; per segment
// [kSegWgs][4] (entries above bin0, candidate count, bin0, entries to take
// from bin0); candidate keys [L], segment p's from p * seg on (a segment's
// candidates keep its order); rounded to 4 words.
constexpr int kCoarse = 64;
__host__ __device__ inline int64_t seg_row_words(int L) {
    return ((int64_t)kSegWgs * (kBins0 + kCoarse) + 4 * kSegWgs + (int64_t)L + 3) & ~(int64_t)3;
}
struct SegRow {
    uint32_t* base;
    int L;
    __device__ uint32_t* hist(int p) const { return base + p * kBins0; }
    __device__ uint32_t* coarse(int p) const { return base + kSegWgs * kBins0 + p * kCoarse; }
    __device__ uint32_t* info(int p) const { return base + kSegWgs * (kBins0 + kCoarse) + 4 * p; }
    __device__ uint32_t* cand_key() const { return info(kSegWgs); }
};

struct SegCoords {
    int r, p, n, lo, hi, seg;
};
__device__ __forceinline__ SegCoords seg_coords(const int32_t* len, int L) {
    SegCoords c;
    c.r = blockIdx.x;
    c.p = blockIdx.y;
    c.n = min(max(len[c.r], 0), L);
    c.seg = (c.n + kSegWgs - 1) / kSegWgs;
    c.lo = min(c.p * c.seg, c.n);
    c.hi = min(c.lo + c.seg, c.n);
    return c;
}

__global__ __launch_bounds__(kSegThreads) void seg_hist_kernel(const float* __restrict__ logits,
                                                               const int32_t* __restrict__ len,
                                                               int32_t* __restrict__ out, uint32_t* __restrict__ ws,
                                                               int L, int K) {
    __shared__ uint32_t hist[kBins0];
    const SegCoords c = seg_coords(len, L);
    const int tid = threadIdx.x;
    if (c.n <= K) {  // every candidate is selected
        if (c.p == 0)
            for (int j = tid; j < K; j += kSegThreads) out[(int64_t)c.r * K + j] = j < c.n ? j : -1;
        return;
    }
    for (int i = tid; i < kBins0; i += kSegThreads) hist[i] = 0;
    __syncthreads();
    const Row row{__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(logits + (int64_t)c.r * L), (short)0,
                                                    c.n * 4, 0x00020000)};
    for (int base = c.lo; base < c.hi; base += kSegKeys * kSegThreads) {
        uint32_t k[kSegKeys];  // one batch of loads in flight
#pragma unroll
        for (int j = 0; j < kSegKeys; ++j) k[j] = row.key(base + j * kSegThreads + tid);
#pragma unroll
        for (int j = 0; j < kSegKeys; ++j)
            if (base + j * kSegThreads + tid < c.hi) atomicAdd(&hist[k[j] >> 20], 1u);
    }
    __syncthreads();
    const SegRow w{ws + c.r * seg_row_words(L), L};
    uint4* dst = reinterpret_cast<uint4*>(w.hist(c.p));
    for (int i = tid; i < kBins0 / 4; i += kSegThreads) dst[i] = reinterpret_cast<const uint4*>(hist)[i];
    if (tid < kCoarse) {  // coarse bin tid = fine bins 64 tid .. 64 tid + 63
        uint32_t sum = 0;
        for (int b = 0; b < kBins0 / kCoarse; ++b) sum += hist[tid * (kBins0 / kCoarse) + b];
        w.coarse(c.p)[tid] = sum;
    }
}

__global__ __launch_bounds__(kSegThreads) void seg_cand_kernel(const float* __restrict__ logits,
                                                               const int32_t* __restrict__ len,
                                                               uint32_t* __restrict__ ws, int L, int K) {
    __shared__ uint32_t tot[kSegThreads / 64];
    __shared__ uint32_t word[3];
    const SegCoords c = seg_coords(len, L);
    if (c.n <= K) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const SegRow w{ws + c.r * seg_row_words(L), L};
    if (tid == 0) word[2] = 0;  // this segment's candidate count
    // this segment's first batch of keys, issued before the histogram reads
    // (it does not depend on them)
    const Row row{__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(logits + (int64_t)c.r * L), (short)0,
                                                    c.n * 4, 0x00020000)};
    uint32_t k[kSegKeys];
#pragma unroll
    for (int j = 0; j < kSegKeys; ++j) k[j] = row.key(c.lo + j * kSegThreads + tid);
    // bin0 in two steps over the row's segments: the coarse bin (key bits
    // 31..26) holding the TOPK-th largest key, then the fine bin within it.
    // Wave 0, lane l: bin 63 - l of each step, counted from the top.
    if (tid < 64) {
        uint32_t v[kSegWgs], sum = 0;
#pragma unroll
        for (int q = 0; q < kSegWgs; ++q) v[q] = w.coarse(q)[kCoarse - 1 - lane];
#pragma unroll
        for (int q = 0; q < kSegWgs; ++q) sum += v[q];
        uint32_t above = wave_incl_scan(sum, lane) - sum;
        const bool cross = above < (uint32_t)K && above + sum >= (uint32_t)K;  // one lane
        const uint64_t m = __ballot(cross);
        const int src = __builtin_ctzll(m);
        const uint32_t cbin = (uint32_t)(kCoarse - 1 - src);
        above = __shfl(above, src);
#pragma unroll
        for (int q = 0; q < kSegWgs; ++q) v[q] = w.hist(q)[cbin * (kBins0 / kCoarse) + (kBins0 / kCoarse - 1 - lane)];
        sum = 0;
#pragma unroll
        for (int q = 0; q < kSegWgs; ++q) sum += v[q];
        uint32_t above2 = above + wave_incl_scan(sum, lane) - sum;
        if (above2 < (uint32_t)K && above2 + sum >= (uint32_t)K) {
            word[0] = cbin * (kBins0 / kCoarse) + (kBins0 / kCoarse - 1 - lane);
            word[1] = above2;
        }
    }
    __syncthreads();
    const uint32_t bin0 = word[0];
    // this segment: count the entries above bin0, append the keys of those in
    // bin0 to the segment's own candidate range
    uint32_t* ck = w.cand_key() + c.lo;
    uint32_t mine_above = 0;
    for (int base = c.lo; base < c.hi; base += kSegKeys * kSegThreads) {
        if (base > c.lo)
#pragma unroll
            for (int j = 0; j < kSegKeys; ++j) k[j] = row.key(base + j * kSegThreads + tid);
#pragma unroll
        for (int j = 0; j < kSegKeys; ++j) {
            const int s = base + j * kSegThreads + tid;
            mine_above += (s < c.hi && (k[j] >> 20) > bin0) ? 1u : 0u;
            const bool hit = s < c.hi && (k[j] >> 20) == bin0;
            const uint64_t m = __ballot(hit);
            if (m) {  // wave-uniform
                uint32_t at = 0;
                if (lane == 0) at = atomicAdd(&word[2], (uint32_t)__popcll(m));
                at = (uint32_t)__builtin_amdgcn_readfirstlane((int)at) + lane_rank(m);
                if (hit) ck[at] = k[j];
            }
        }
    }
    mine_above = wave_sum(mine_above);
    __syncthreads();  // tot is reused
    if (lane == 0) tot[tid >> 6] = mine_above;
    __syncthreads();
    if (tid == 0) {
        uint32_t a = 0;
        for (int v = 0; v < kSegThreads / 64; ++v) a += tot[v];
        *reinterpret_cast<uint4*>(w.info(c.p)) = uint4{a, word[2], bin0, (uint32_t)K - word[1]};
    }
}

// Exclusive prefix (in thread order) and total over the workgroup of a
// per-thread count.  Uses tot[kSegThreads / 64] of LDS.
__device__ __forceinline__ void block_prefix(uint32_t c, uint32_t* tot, uint32_t& before, uint32_t& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t incl = wave_incl_scan(c, lane);
    if (lane == 63) tot[wave] = incl;
    __syncthreads();
    before = incl - c;
    total = 0;
#pragma unroll
    for (int w = 0; w < kSegThreads / 64; ++w) {
        const uint32_t t = tot[w];
        if (w < wave) before += t;
        total += t;
    }
    __syncthreads();  // tot is rewritten by the next call
}

__global__ __launch_bounds__(kSegThreads) void seg_emit_kernel(const float* __restrict__ logits,
                                                               const int32_t* __restrict__ len,
                                                               int32_t* __restrict__ out,
                                                               const uint32_t* __restrict__ ws, int L, int K) {
    __shared__ uint32_t ck[kSegCandCap];
    __shared__ uint32_t hist[kBins0];
    __shared__ uint32_t gt[kSegWgs], eq[kSegWgs];
    __shared__ uint32_t above[kSegWgs], cbase[kSegWgs + 1];
    __shared__ uint32_t tot[kSegThreads / 64];
    __shared__ uint32_t word[4];
    const SegCoords c = seg_coords(len, L);
    if (c.n <= K) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const SegRow w{const_cast<uint32_t*>(ws) + c.r * seg_row_words(L), L};
    // One round trip: every segment's info, the first kWin candidates of every
    // segment's range (read before their counts are known) and this
    // segment's first batch of keys.
    constexpr int kWin = 128;                             // candidates per segment
    constexpr int kWinPer = kSegWgs * kWin / kSegThreads;  // window slots per thread
    const Row row{__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(logits + (int64_t)c.r * L), (short)0,
                                                    c.n * 4, 0x00020000)};
    uint32_t h[kSegKeys];
#pragma unroll
    for (int j = 0; j < kSegKeys; ++j) h[j] = row.key(c.lo + kSegKeys * tid + j);
    uint4 info = uint4{0, 0, 0, 0};
    if (tid < kSegWgs) info = *reinterpret_cast<const uint4*>(w.info(tid));
    // slot m of this thread: segment wq, index wi
    const int wq = tid / (kWin / kWinPer);
    uint32_t win_k[kWinPer];
#pragma unroll
    for (int m = 0; m < kWinPer; ++m)
        win_k[m] = w.cand_key()[min(wq * c.seg + (tid % (kWin / kWinPer)) + m * (kWin / kWinPer), L - 1)];
    if (tid < kSegWgs) {  // every segment's (entries above bin0, candidate count), bin0 and the entries to take
        above[tid] = info.x;
        cbase[tid] = info.y;
        if (tid == 0) {
            word[0] = info.z;
            word[1] = info.w;
        }
        gt[tid] = eq[tid] = 0;
    }
    for (int i = tid; i < kBins0; i += kSegThreads) hist[i] = 0;
    __syncthreads();
    const bool windows = __syncthreads_and(tid >= kSegWgs || info.y <= (uint32_t)kWin);
    if (tid == 0) {  // candidate counts -> offsets of the compacted list
        uint32_t acc = 0;
        for (int q = 0; q < kSegWgs; ++q) {
            const uint32_t n_q = cbase[q];
            cbase[q] = acc;
            acc += n_q;
        }
        cbase[kSegWgs] = acc;
    }
    __syncthreads();
    const uint32_t bin0 = word[0];
    uint32_t need = word[1];
    const int ncand = (int)cbase[kSegWgs];
    const bool in_lds = ncand <= kSegCandCap;
    // candidate i lives in segment q's range: index q * seg + (i - cbase[q])
    auto src_index = [&](int i) -> int {
        int q = 0;
#pragma unroll
        for (int t = 1; t < kSegWgs; ++t) q += (uint32_t)i >= cbase[t] ? 1 : 0;
        return q * c.seg + (i - (int)cbase[q]);
    };
    if (windows) {  // every candidate came with the first round trip
        const uint32_t nq = cbase[wq + 1] - cbase[wq];
#pragma unroll
        for (int m = 0; m < kWinPer; ++m) {
            const uint32_t wi = (uint32_t)(tid % (kWin / kWinPer) + m * (kWin / kWinPer));
            if (wi < nq) ck[cbase[wq] + wi] = win_k[m];
        }
    } else if (in_lds) {
        for (int i = tid; i < ncand; i += kSegThreads) ck[i] = w.cand_key()[src_index(i)];
    }
    __syncthreads();
    // The candidates are read from LDS, or (more than kSegCandCap of them) from
    // the workspace: two instantiations, so the LDS one holds no global load.
    auto resolve = [&](auto from_lds) -> uint32_t {
    constexpr bool kLds = decltype(from_lds)::value;
    auto key_at = [&](int i) -> uint32_t {
        if constexpr (kLds) return ck[i];
        else return w.cand_key()[src_index(i)];
    };

    // ---- T: the need-th largest candidate key (all share bits 31..20 = bin0):
    // bits 19..8 from a 4096-bin histogram, then bits 7..0 from 256 bins
    for (int i = tid; i < ncand; i += kSegThreads) atomicAdd(&hist[(key_at(i) >> 8) & (kBins0 - 1)], 1u);
    __syncthreads();
    {
        // thread tid owns bins kBins0 - 1 - 16 tid - j (j = 0..15), counted from the top
        uint32_t cnt[16], mine = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            cnt[j] = hist[kBins0 - 1 - 16 * tid - j];
            mine += cnt[j];
        }
        uint32_t before, total;
        block_prefix(mine, tot, before, total);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (before < need && before + cnt[j] >= need) {  // exactly one (thread, j) crosses
                word[2] = (uint32_t)(kBins0 - 1 - 16 * tid - j);
                word[3] = before;
            }
            before += cnt[j];
        }
    }
    __syncthreads();
    const uint32_t pre24 = (bin0 << 12) | word[2];  // key bits 31..8 of T
    need -= word[3];
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < ncand; i += kSegThreads) {
        const uint32_t u = key_at(i);
        if ((u >> 8) == pre24) atomicAdd(&hist[u & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {  // four bins per lane from the top
        uint32_t cc[4], sum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            cc[j] = hist[255 - (4 * lane + j)];
            sum += cc[j];
        }
        uint32_t a = wave_incl_scan(sum, lane) - sum;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (a < need && a + cc[j] >= need) word[2] = (uint32_t)(255 - (4 * lane + j));
            a += cc[j];
        }
    }
    __syncthreads();
    const uint32_t thr = (pre24 << 8) | word[2];

    // ---- per segment: candidates above T and equal to T (wave ballots); ties
    // go to the lowest s
    {
        // The list holds the segments in order, so candidate i belongs to the
        // segment q with cbase[q] <= i < cbase[q + 1].
        uint32_t ngt[kSegWgs] = {};
        for (int base = 0; base < ncand; base += kSegThreads) {
            const int i = base + tid;
            const uint32_t u = i < ncand ? key_at(i) : 0u;
            int q = -1;
            if (i < ncand) {
                q = 0;
#pragma unroll
                for (int t = 1; t < kSegWgs; ++t) q += (uint32_t)i >= cbase[t] ? 1 : 0;
                if (u == thr) atomicAdd(&eq[q], 1u);  // rare
            }
#pragma unroll
            for (int qq = 0; qq < kSegWgs; ++qq) ngt[qq] += (uint32_t)__popcll(__ballot(q == qq && u > thr));
        }
        if (lane == 0)
#pragma unroll
            for (int qq = 0; qq < kSegWgs; ++qq)
                if (ngt[qq]) atomicAdd(&gt[qq], ngt[qq]);
    }
    __syncthreads();
    return thr;
    };
    const uint32_t thr = in_lds ? resolve(std::true_type{}) : resolve(std::false_type{});
    if (tid == 0) {  // offsets: segments in order, ties to the earliest
        uint32_t gt_all = 0;
        for (int q = 0; q < kSegWgs; ++q) gt_all += gt[q];
        uint32_t off = 0, left = word[1] - gt_all;  // entries equal to T to take
        for (int q = 0; q < kSegWgs; ++q) {
            const uint32_t take = min(eq[q], left);
            left -= take;
            if (q == c.p) {
                word[2] = off;
                word[3] = take;
            }
            off += above[q] + gt[q] + take;
        }
    }
    __syncthreads();
    uint32_t pos = word[2];
    const uint32_t take = word[3];

    // ---- this segment's selected s, ascending: kSegKeys consecutive entries per thread
    int32_t* dst = out + (int64_t)c.r * K;
    uint32_t ties = 0;
    for (int base = c.lo; base < c.hi; base += kSegKeys * kSegThreads) {
        const int s0 = base + kSegKeys * tid;
        if (base > c.lo)
#pragma unroll
            for (int j = 0; j < kSegKeys; ++j) h[j] = row.key(s0 + j);
        uint32_t gtm = 0, eqm = 0;
#pragma unroll
        for (int j = 0; j < kSegKeys; ++j) {
            const bool ok = s0 + j < c.hi;
            gtm |= (ok && h[j] > thr) ? 1u << j : 0u;
            eqm |= (ok && h[j] == thr) ? 1u << j : 0u;
        }
        uint32_t selm = gtm, eq_total = 0;
        if (__syncthreads_or(eqm != 0u)) {  // rare: ties in this batch
            uint32_t eq_before;
            block_prefix((uint32_t)__popc(eqm), tot, eq_before, eq_total);
            uint32_t rank = ties + eq_before;
#pragma unroll
            for (int j = 0; j < kSegKeys; ++j)
                if ((eqm >> j) & 1u) {
                    if (rank < take) selm |= 1u << j;
                    ++rank;
                }
        }
        uint32_t sel_before, sel_total;
        block_prefix((uint32_t)__popc(selm), tot, sel_before, sel_total);
        uint32_t at = pos + sel_before;
#pragma unroll
        for (int j = 0; j < kSegKeys; ++j)
            if ((selm >> j) & 1u) dst[at++] = s0 + j;
        pos += sel_total;
        ties += eq_total;
    }
}

template <int HI, int KS>
int launch_logits(const IndexerParams& p, dim3 grid, hipStream_t stream) {
    hipLaunchKernelGGL((indexer_logits_kernel<HI, KS>), grid, dim3(256), 0, stream, p);
    return (int)hipGetLastError();
}

}  // namespace

int launch_indexer_logits(const IndexerParams& p, hipStream_t stream) {
    const dim3 grid((unsigned)(p.B * p.tgroups), (unsigned)((p.ntiles + p.tiles_per_wg - 1) / p.tiles_per_wg));
    if (p.HI == 64) {
        if (p.ks == 1) return launch_logits<64, 1>(p, grid, stream);
        if (p.ks == 2) return launch_logits<64, 2>(p, grid, stream);
        if (p.ks == 4) return launch_logits<64, 4>(p, grid, stream);
    } else if (p.HI == 32) {
        if (p.ks == 1) return launch_logits<32, 1>(p, grid, stream);
        if (p.ks == 2) return launch_logits<32, 2>(p, grid, stream);
        if (p.ks == 4) return launch_logits<32, 4>(p, grid, stream);
    }
    return (int)hipErrorInvalidValue;
}

int64_t indexer_topk_ws_bytes(int rows, int L) {
    if (rows > kSegMaxRows) return 0;
    return (int64_t)rows * seg_row_words(L) * 4;
}

int launch_indexer_topk_seg(const float* logits, const int32_t* len, int32_t* indices, void* ws, int rows, int L,
                            int topk, hipStream_t stream) {
    uint32_t* w = static_cast<uint32_t*>(ws);
    const dim3 grid((unsigned)rows, (unsigned)kSegWgs);
    hipLaunchKernelGGL(seg_hist_kernel, grid, dim3(kSegThreads), 0, stream, logits, len, indices, w, L, topk);
    hipLaunchKernelGGL(seg_cand_kernel, grid, dim3(kSegThreads), 0, stream, logits, len, w, L, topk);
    hipLaunchKernelGGL(seg_emit_kernel, grid, dim3(kSegThreads), 0, stream, logits, len, indices,
                       static_cast<const uint32_t*>(w), L, topk);
    return (int)hipGetLastError();
}

int launch_indexer_topk(const float* logits, const int32_t* len, int32_t* indices, int rows, int L, int topk,
                        hipStream_t stream) {
    hipLaunchKernelGGL(indexer_topk_kernel, dim3((unsigned)rows), dim3(kTopkThreads), 0, stream, logits, len,
                       indices, L, topk);
    return (int)hipGetLastError();
}

}  // namespace dsa
