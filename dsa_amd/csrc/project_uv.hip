// W_UV output projection: the step after the attention in MLA's absorbed form.
// The attention returns each head's output in the 512-wide latent space; the
// model maps it to the value head dimension with that head's slice of the
// kv up-projection (DeepSeek-V3.2-Exp inference/model.py, MLA.forward, absorb
// branch: x = einsum("bshc,hdc->bshd", x, wkv_b[:, -v_head_dim:]); the
// reference names the model's own scale and layout at README.md:81-83 and
// FAIRNESS_AUDIT.md:28):
//
//   out_v[t, h, d] = bf16( sum_{c < 512} lat[t, h, c] * W[h, d, c] ),   d < dv
//
// lat [T, H, 512] bf16 (the attention output), W [H, dv, 512] bf16 with any
// head stride (a slice of wkv_b's rows needs no copy), out_v [T, H, dv] bf16.
//
// One kernel, two sources for the latent tile:
//  * copy  -- lat is read from memory (dsa_project_uv);
//  * merge -- lat is the split merge of FP32 partials, computed into LDS with
//             merge_math.h's arithmetic, so it holds the bits dsa_merge would
//             have written; the 512-wide output never reaches HBM and the
//             merge's second launch disappears (dsa_merge_uv).
// Either way the projection below is the same code, so dsa_merge_uv's out_v
// equals dsa_project_uv(dsa_merge(...)) bit for bit.
//
// Both kernels run the same projection routine (mma_tile): wave w owns
// NJ 16-row d tiles of its workgroup's d range and holds their weight rows in
// registers (A operand: 16 d x 32 c per k-step, 16 k-steps, 64 VGPRs a tile,
// read from memory once per workgroup); the latent tile is the B operand
// (32 c x 16 tokens) from LDS; D = out_v^T (16 d x 16 tokens), so each lane
// ends with 4 consecutive d of one token: one 8-byte store.  Per output
// element the chain is the same 16 MFMAs in the same order in both kernels,
// which is what makes merge_uv's result equal project_uv(merge) bit for bit.
//
// * project_kernel<NJ>: workgroup = (head, chunk of tokens, d part).  The
//   weights are loaded once; the chunk is walked in tiles of 32 tokens
//   through four LDS buffers, the latent rows loaded straight into LDS
//   (buffer_load ... lds), three tiles in flight while one is multiplied,
//   one LDS-only barrier per tile.  Every latent byte is read from HBM once.
//   The B fragments are read from LDS in groups of 8, one group ahead of the
//   MFMAs that use them.
// * merge_uv_kernel<NJ, BATCH>: workgroup = (head, 16 tokens, d part).  The
//   merge fills the tile: each thread merges 32 / BATCH (16 / BATCH with two
//   weight tiles; 1 to 8) units of 4 columns of one token row, the row's
//   max, weights and sum once per thread, every split load in flight at
//   once, the batch width matched to the split count.
//
// LDS tile: latent rows of 1 KiB; 16-byte chunk c of row t sits at chunk
// c ^ (t & 15), so the 16 rows one B-operand read touches hit distinct banks.
#include <hip/hip_runtime.h>
#include <float.h>
#include <stdint.h>

#include "kernels.h"
#include "merge_math.h"

namespace dsa {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef merge_f32x4 f32x4;

constexpr int kThreads = 256;
constexpr int kKSteps = 16;  // 512 latent columns / 32 per MFMA

struct UvArgs {
    const uint16_t* lat;     // copy source [T, H, 512]
    const float* part_o;     // merge source [T, nsplit, H, 512]
    const float* part_m;     // [T, nsplit, H]
    const float* part_l;
    float* out_max;          // [T, H] (merge source only)
    float* out_sum;
    const uint16_t* w;       // [H, dv, 512] with head stride w_head_stride elements
    int64_t w_head_stride;
    uint16_t* out_v;         // [T, H, dv]
    int T, H, dv, nsplit;
    int nchunk, chunk_tokens, dsplit;  // launch shape
};

__device__ __forceinline__ uint32_t tile_off(int t, int chunk) {
    return (uint32_t)t * 1024u + ((uint32_t)(chunk ^ (t & 15)) << 4);
}

// blockIdx -> (head, token chunk, d part).  With H a multiple of 8, the
// workgroups of one head run on one XCD (workgroups are dealt to the 8 XCDs
// round robin), so the head's weights are fetched into that XCD's L2 once.
__device__ __forceinline__ void block_coords(const UvArgs& a, int& h, int& chunk, int& dp) {
    const int bid = blockIdx.x;
    const int per_head = a.nchunk * a.dsplit;
    int slot;
    if ((a.H & 7) == 0) {
        slot = bid >> 3;
        const int hb = slot / per_head;
        h = hb * 8 + (bid & 7);
        slot -= hb * per_head;
    } else {
        h = bid / per_head;
        slot = bid - h * per_head;
    }
    chunk = slot / a.dsplit;
    dp = slot - chunk * a.dsplit;
}

// Weight rows of this wave's NJ d tiles: tile q is d rows
// 16 * (dp * 4 * NJ + 4 * q + wave) + [0, 16).
template <int NJ>
__device__ __forceinline__ void load_weights(bf16x8 (&wf)[NJ][kKSteps], const UvArgs& a, int h, int dp) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint16_t* wh = a.w + (int64_t)h * a.w_head_stride + 8 * (lane >> 4);
#pragma unroll
    for (int q = 0; q < NJ; ++q) {
        const uint16_t* wrow = wh + (int64_t)(16 * (dp * 4 * NJ + 4 * q + wave) + (lane & 15)) * 512;
#pragma unroll
        for (int k = 0; k < kKSteps; ++k) wf[q][k] = *reinterpret_cast<const bf16x8*>(wrow + 32 * k);
    }
}

// D = out_v^T of one latent tile: NT token tiles of 16, this wave's NJ d
// tiles.  B fragments are read from LDS in groups of KG k-steps (8
// fragments), the next group's reads issued before the current group's MFMAs.
template <int NT, int NJ>
__device__ __forceinline__ void mma_tile(const uint8_t* tile, const bf16x8 (&wf)[NJ][kKSteps], f32x4 (&acc)[NJ][NT]) {
    const int lane = threadIdx.x & 63;
    const int n16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int q = 0; q < NJ; ++q)
#pragma unroll
        for (int i = 0; i < NT; ++i) acc[q][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int KG = 8 / NT;
    bf16x8 lf[2][KG][NT];
    auto read_group = [&](bf16x8 (&dst)[KG][NT], int kg) {
#pragma unroll
        for (int kk = 0; kk < KG; ++kk)
#pragma unroll
            for (int i = 0; i < NT; ++i)
                dst[kk][i] = *reinterpret_cast<const bf16x8*>(tile + tile_off(16 * i + n16, 4 * (kg * KG + kk) + g));
    };
    // The scheduling barriers keep each group's reads ahead of the MFMAs of
    // the group before (the scheduler would otherwise sink every read next
    // to its first use and wait out the LDS latency at each k-step).
    read_group(lf[0], 0);
#pragma unroll
    for (int kg = 0; kg < kKSteps / KG; ++kg) {
        if (kg + 1 < kKSteps / KG) read_group(lf[(kg + 1) & 1], kg + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < KG; ++kk)
#pragma unroll
            for (int i = 0; i < NT; ++i)
#pragma unroll
                for (int q = 0; q < NJ; ++q)
                    acc[q][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[q][kg * KG + kk], lf[kg & 1][kk][i],
                                                                        acc[q][i], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

__device__ __forceinline__ merge_bf16x4 to_bf16(f32x4 v) {
    merge_bf16x4 o;
    o[0] = (__bf16)v[0];
    o[1] = (__bf16)v[1];
    o[2] = (__bf16)v[2];
    o[3] = (__bf16)v[3];
    return o;
}

// Lane: d = 16 (tile) + 4 g + r (r < 4) of token 16 i + n16.  Column offset
// of this wave's d tile q within a token's dv values.
template <int NJ>
__device__ __forceinline__ int d_col(int dp, int q) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return 16 * (dp * 4 * NJ + 4 * q + wave) + 4 * (lane >> 4);
}

// Barrier over LDS writes only: outstanding global loads stay in flight
// across it (__syncthreads would wait for them).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((__vector_size__(2 * sizeof(unsigned))));

// One 1 KiB latent row into LDS with buffer_load_dwordx4 ... lds: lane l
// fetches chunk l ^ sw of the row, which lands at lds + 16 l, so logical
// chunk c sits at c ^ sw (tile_off's layout).  The row address and lds are
// wave-uniform.  Issued as inline asm, so the compiler neither waits for it
// at its own waits nor turns it into a branch; completion is tracked with
// wait_vmcnt.
__device__ __forceinline__ void row_to_lds(uint32_t lds, const uint16_t* row, uint32_t voff) {
    const uint64_t addr = reinterpret_cast<uint64_t>(row);
    i32x4 rsrc;
    rsrc[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
    rsrc[1] = __builtin_amdgcn_readfirstlane((int)((addr >> 32) & 0xffff));
    rsrc[2] = 1024;
    rsrc[3] = 0x00020000;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
#pragma clang diagnostic pop
}

constexpr int kPTB = 32;   // tokens per tile of the copy path
constexpr int kPBuf = 4;   // LDS buffers: three tiles in flight while one is multiplied

template <int NJ>
__global__ __launch_bounds__(kThreads) void project_kernel(UvArgs a) {
    constexpr int TB = kPTB, NT = TB / 16, RPW = TB / 4;  // rows per wave per tile
    constexpr int L = RPW, NS = NT * NJ;                    // loads / stores per lane per tile
    __shared__ __attribute__((aligned(16))) uint8_t tiles[kPBuf][TB * 1024];
    int h, chunk, dp;
    block_coords(a, h, chunk, dp);
    const int c0 = chunk * a.chunk_tokens;
    const int c1 = min(a.T, c0 + a.chunk_tokens);
    const int ntiles = (c1 - c0 + TB - 1) / TB;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);

    bf16x8 wf[NJ][kKSteps];
    load_weights<NJ>(wf, a, h, dp);

    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)&tiles[0][0];
    // This wave's rows of tile i: wave + 4 r.  Rows past the chunk's end load
    // the chunk's last row again (in bounds): they feed only D columns that
    // are never stored.
    auto issue = [&](int i) {
        const int t0 = c0 + i * TB;
        const uint32_t buf = lds0 + (uint32_t)(i % kPBuf) * (TB * 1024);
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int tt = wave + 4 * r;
            const int src = min(t0 + tt, c1 - 1);
            row_to_lds(buf + (uint32_t)tt * 1024u, a.lat + ((int64_t)src * a.H + h) * 512,
                       16u * ((uint32_t)lane ^ (uint32_t)(tt & 15)));
        }
    };
    for (int i = 0; i < 3 && i < ntiles; ++i) issue(i);

    const int n16 = lane & 15;
    for (int i = 0; i < ntiles; ++i) {
        // Tile i's loads are complete once no more than the loads and
        // stores issued after them are outstanding: tiles i + 1 and i + 2
        // (2 L) and the stores of the last min(i, 3) tiles (NS each).
        if (i + 2 < ntiles) {
            if (i == 0) wait_vmcnt<2 * L>();
            else if (i == 1) wait_vmcnt<2 * L + NS>();
            else if (i == 2) wait_vmcnt<2 * L + 2 * NS>();
            else wait_vmcnt<2 * L + 3 * NS>();
        } else {
            wait_vmcnt<0>();
        }
        lds_barrier();  // every wave's rows of tile i are in; buffer (i + 3) % 4 is free
        if (i + 3 < ntiles) issue(i + 3);
        f32x4 acc[NJ][NT];
        mma_tile<NT, NJ>(tiles[i % kPBuf], wf, acc);
        // Exactly NS buffer stores per lane: a token past the chunk's end
        // gets an offset past the descriptor's range, which drops the store.
        const int t0 = c0 + i * TB;
        const int ntok = min(TB, c1 - t0);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            a.out_v + ((int64_t)t0 * a.H + h) * a.dv, (short)0, ((ntok - 1) * a.H + 1) * a.dv * 2, 0x00020000);
#pragma unroll
        for (int ti = 0; ti < NT; ++ti) {
            const int tt = 16 * ti + n16;
#pragma unroll
            for (int q = 0; q < NJ; ++q) {
                const int off = tt < ntok ? (tt * a.H * a.dv + d_col<NJ>(dp, q)) * 2 : 0x7ffffff0;
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, to_bf16(acc[q][ti])), rs, off, 0, 0);
            }
        }
    }
}

template <int NJ, int BATCH>
__global__ __launch_bounds__(kThreads) void merge_uv_kernel(UvArgs a) {
    constexpr int TB = 16;
    // Units of 4 columns per thread per pass (a power of two dividing 128):
    // the split loads of a pass in registers stay near 128 VGPRs (64 with
    // the second weight tile).
    constexpr int BUDGET = NJ == 2 ? 16 : 32;
    constexpr int NU = BUDGET / BATCH < 1 ? 1 : BUDGET / BATCH < 8 ? BUDGET / BATCH : 8;
    __shared__ __attribute__((aligned(16))) uint8_t tile[TB * 1024];
    int h, blk, dp;
    block_coords(a, h, blk, dp);
    const int t0 = blk * TB;
    const int ntok = min(TB, a.T - t0);

    bf16x8 wf[NJ][kKSteps];

    // A thread merges NU units of 4 columns of one token row (its row's max,
    // weights and sum computed once): G = 128 / NU threads per row, 2 NU rows
    // per pass, unit r of thread c of a row at columns 4 (c + G r); each half
    // of a wave (G = 32) reads 512 contiguous bytes per load.  Rows past ntok
    // are left unwritten: they feed only the D columns of tokens that are
    // never stored (an MFMA's column n reads column n of B only).
    constexpr int G = 128 / NU;
    const int rsub = threadIdx.x / G, cg = threadIdx.x % G;
    load_weights<NJ>(wf, a, h, dp);
    for (int tt = rsub; tt < ntok; tt += kThreads / G) {
        const int64_t base = (int64_t)(t0 + tt) * a.nsplit * a.H + h;
        int col[NU];
#pragma unroll
        for (int r = 0; r < NU; ++r) col[r] = 4 * (cg + G * r);
        f32x4 acc[NU];
        float m, l;
        merge_row<NU, BATCH>(a.part_o, a.part_m, a.part_l, base, col, a.H, a.nsplit, acc, m, l);
#pragma unroll
        for (int r = 0; r < NU; ++r) {
            const int c = cg + G * r;
            *reinterpret_cast<merge_bf16x4*>(tile + tile_off(tt, c >> 1) + ((c & 1) << 3)) = merge_finish(acc[r], l);
        }
        if (cg == 0 && dp == 0) {
            const int64_t orow = (int64_t)(t0 + tt) * a.H + h;
            a.out_max[orow] = m;
            a.out_sum[orow] = l;
        }
    }
    lds_barrier();
    f32x4 acc[NJ][1];
    mma_tile<1, NJ>(tile, wf, acc);
    const int tt = threadIdx.x & 15;
    if (tt < ntok) {
        uint16_t* row = a.out_v + ((int64_t)(t0 + tt) * a.H + h) * a.dv;
#pragma unroll
        for (int q = 0; q < NJ; ++q) *reinterpret_cast<merge_bf16x4*>(row + d_col<NJ>(dp, q)) = to_bf16(acc[q][0]);
    }
}

// d tiles per wave and d parts: two tiles per wave (NJ 2) when that still
// leaves one workgroup per CU, else one, the d range split so that each
// part is 4 * NJ tiles.
void d_shape(int dv, int64_t wgs, int& nj, int& dsplit) {
    const int ndt = dv / 16;  // 4, 8, 12 or 16
    nj = (ndt % 8 == 0 && wgs * (ndt / 8) >= 256) ? 2 : 1;
    dsplit = ndt / (4 * nj);
}

// Launch shape of one call (mirrored by the host's launch descriptors).
void uv_shape(int T, int H, int dv, bool merge, int& tb, int& nj, int& dsplit, int& nchunk, int& chunk_tokens) {
    if (merge) {
        tb = 16;
        nchunk = (T + 15) / 16;
        chunk_tokens = 16;
        d_shape(dv, (int64_t)H * nchunk, nj, dsplit);
        return;
    }
    // Tiles of kPTB tokens; the chunks of a head aim at one workgroup per CU
    // overall.
    tb = kPTB;
    const int ntiles = (T + tb - 1) / tb;
    int64_t want = (256 + H - 1) / H;  // chunks per head
    d_shape(dv, (int64_t)H * ntiles, nj, dsplit);
    want = (want + dsplit - 1) / dsplit;
    const int per = (int)((ntiles + want - 1) / want);  // tiles per chunk
    chunk_tokens = per * tb;
    nchunk = (ntiles + per - 1) / per;
}

int launch_uv(UvArgs a, bool merge, hipStream_t stream) {
    int tb, nj;
    uv_shape(a.T, a.H, a.dv, merge, tb, nj, a.dsplit, a.nchunk, a.chunk_tokens);
    const int64_t grid = (int64_t)a.H * a.nchunk * a.dsplit;
    const dim3 g((unsigned)grid), b(kThreads);
    if (merge) {
        const int s = a.nsplit;
        if (nj == 2) {
            if (s <= 2) hipLaunchKernelGGL((merge_uv_kernel<2, 2>), g, b, 0, stream, a);
            else if (s <= 4) hipLaunchKernelGGL((merge_uv_kernel<2, 4>), g, b, 0, stream, a);
            else if (s <= 8) hipLaunchKernelGGL((merge_uv_kernel<2, 8>), g, b, 0, stream, a);
            else hipLaunchKernelGGL((merge_uv_kernel<2, kMergeBatch>), g, b, 0, stream, a);
        } else {
            if (s <= 2) hipLaunchKernelGGL((merge_uv_kernel<1, 2>), g, b, 0, stream, a);
            else if (s <= 4) hipLaunchKernelGGL((merge_uv_kernel<1, 4>), g, b, 0, stream, a);
            else if (s <= 8) hipLaunchKernelGGL((merge_uv_kernel<1, 8>), g, b, 0, stream, a);
            else hipLaunchKernelGGL((merge_uv_kernel<1, kMergeBatch>), g, b, 0, stream, a);
        }
    } else if (nj == 2) {
        hipLaunchKernelGGL((project_kernel<2>), g, b, 0, stream, a);
    } else {
        hipLaunchKernelGGL((project_kernel<1>), g, b, 0, stream, a);
    }
    return (int)hipGetLastError();
}

}  // namespace

int launch_project_uv(const uint16_t* lat, const uint16_t* w, int64_t w_head_stride, uint16_t* out_v, int tokens,
                      int H, int dv, hipStream_t stream) {
    UvArgs a{};
    a.lat = lat;
    a.w = w;
    a.w_head_stride = w_head_stride;
    a.out_v = out_v;
    a.T = tokens;
    a.H = H;
    a.dv = dv;
    return launch_uv(a, false, stream);
}

int launch_merge_uv(const float* part_o, const float* part_m, const float* part_l, const uint16_t* w,
                    int64_t w_head_stride, uint16_t* out_v, float* out_max, float* out_sum, int tokens, int H,
                    int nsplit, int dv, hipStream_t stream) {
    UvArgs a{};
    a.part_o = part_o;
    a.part_m = part_m;
    a.part_l = part_l;
    a.out_max = out_max;
    a.out_sum = out_sum;
    a.w = w;
    a.w_head_stride = w_head_stride;
    a.out_v = out_v;
    a.T = tokens;
    a.H = H;
    a.dv = dv;
    a.nsplit = nsplit;
    return launch_uv(a, true, stream);
}

}  // namespace dsa
