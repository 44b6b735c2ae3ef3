// Sparse-MLA attention forward for gfx950 (MI355X).
//
// One workgroup (4 waves) owns (token, KV split, head group).  It gathers the
// selected 576-wide rows (kv[:512] ++ k_rope[:64]) straight from HBM into an
// LDS ring with buffer_load_dwordx4 ... lds (no VGPR staging); every wave then
// computes, for its slice of heads and rows,
//
//   S^T[row, head] = K[row, :576] . Q[head, :576]       A = K from LDS, B = Q in VGPRs
//   softmax over rows in registers (log2 units, FP32 state)
//   O^T[col, head] += V^T[col, row] . P^T[row, head]    A = V read with ds_read_b64_tr_b16,
//                                                        B = P in VGPRs
//
// S^T puts the head on the lane index, which is exactly the lane layout the
// PV B operand needs, so P never leaves registers; all heads of the group
// share one gathered tile.  Two variants:
//
//   wide   -- v_mfma_f32_32x32x16_bf16, 32 heads per wave (Q: 144 VGPRs,
//             O: 256 accumulators): 4 head-waves = 128 heads per workgroup on
//             32-row tiles (4-stage ring), or 2 head-waves x 2 row-waves = 64
//             heads on 64-row tiles.
//   narrow -- v_mfma_f32_16x16x32_bf16, 16 heads per wave: 64, 32 or 16 heads
//             per workgroup with 1, 2 or 4 row-waves on 64-row tiles.
//
// Math follows the reference workspace kernel (dsa/workspace.py:242-390):
// running max initialised to -FLT_MAX (:68), scores scaled and masked by the
// index (:252-257), FP32 sum of the FP32 exponentials, P rounded to bf16
// (RNE) before PV (:270-272), FP32 accumulation, and for split > 1 the
// unnormalised FP32 numerator plus (max, sum) partials (:379-385).  Scores are
// carried in log2 units (x * scale * log2(e); the reference's scale is 1/24)
// so that every exponential is one v_exp_f32; max/sum leave the kernel in
// natural units.
#include <hip/hip_runtime.h>
#include <type_traits>
#include <float.h>
#include <stdint.h>

#include "kernels.h"
#include "merge_math.h"
#include "../../include/dsa_mi355x.h"

namespace dsa {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;

// log2(e) / 24: multiplying the raw QK dot product by this gives the score in
// log2 units, so exp(score - max) == exp2(x - x_max).
constexpr float kLn2 = 0.69314718055994531f;
// P is formed against a reference max m_ref fixed at the first tile with a
// valid row and is clamped at 2^kRestartLog2; a head whose running max exceeds
// m_ref by more than that makes the workgroup recompute its range once with
// m_ref = the exact max.  The O accumulators therefore never see VALU work
// inside the tile loop (a rescale there would move every accumulator between
// AGPRs and VGPRs on every tile).  bf16 P keeps its relative precision at any
// scale and FP32 O, l stay far from overflow (2^64 * TOPK).
constexpr float kRestartLog2 = 64.0f;

// ------------------------------------------------------------ ring layout
// 4 waves per workgroup.  LDS: NSTAGE stages of [BN rows][1024 B kv] then
// [BN rows][128 B rope], then the slot indices of the workgroup, then one
// flag word (second-pass vote of the wide variant).
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
// ---------------------------------------------------------------- LDS access
template <typename T>
__device__ __forceinline__ T lds_load(uint32_t addr) {
    return *reinterpret_cast<__attribute__((address_space(3))) T*>(addr);
}
template <typename T>
__device__ __forceinline__ void lds_store(uint32_t addr, T v) {
    *reinterpret_cast<__attribute__((address_space(3))) T*>(addr) = v;
}
// ds_read_b64_tr_b16: within each 16-lane group, lane l supplies the address
// of 4 consecutive bf16 of "row" l/4, columns 4*(l%4)..+3 of a 4x16 block;
// lane n receives column n of that block (rows 0..3).
__device__ __forceinline__ bf16x4 lds_load_tr(uint32_t addr) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        reinterpret_cast<__attribute__((address_space(3))) bf16x4*>(addr));
}

// Barrier that makes this workgroup's LDS writes visible without waiting for
// outstanding global loads (the gather ring stays in flight across it).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef int rsrc_t __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + bytes) (gfx9 descriptor: no stride,
// 32-bit byte offsets).  All fields are wave-uniform.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    rsrc_t r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff));
    r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
    r[3] = 0x00020000;
    return r;
}

// Gathers write LDS with buffer_load_dwordx4 ... lds: lane l's 16 bytes land
// at m0 + 16*l.  They are issued as inline asm so the compiler does not
// serialise later LDS reads behind them; completion is tracked with
// Ring::wait_tile().  m0 and the buffer descriptors are wave-uniform by
// construction.
//
// One kv row: a 1 KiB descriptor at the row's 64-bit address (so the kv
// pool has no 4 GiB limit), lane l loading bytes (16*l) ^ xor16 of it.  The
// XOR is part of the asm so no per-row lane offset is ever kept live.
__device__ __forceinline__ rsrc_t row_rsrc(const char* base, uint32_t row) {
    const uint64_t a = reinterpret_cast<uint64_t>(base) + ((uint64_t)row << 10);
    rsrc_t r;
    r[0] = (int)(uint32_t)a;
    r[1] = (int)((a >> 32) & 0xffff);
    r[2] = 1024;
    r[3] = 0x00020000;
    return r;
}
__device__ __forceinline__ void gather_row(uint32_t lds_base, rsrc_t rsrc, uint32_t lane16, uint32_t xor16) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    uint32_t voff;
    asm volatile(
        "v_xor_b32 %0, %1, %2\n\t"
        "s_mov_b32 m0, %3\n\t"
        "buffer_load_dwordx4 %0, %4, 0 offen lds"
        : "=&v"(voff)
        : "s"(xor16), "v"(lane16), "s"(__builtin_amdgcn_readfirstlane(lds_base)), "s"(rsrc)
        : "memory", "m0");
#pragma clang diagnostic pop
}
// Arbitrary per-lane byte offsets (rope rows: 8 rows per instruction).
__device__ __forceinline__ void gather_lanes(uint32_t lds_base, rsrc_t rsrc, uint32_t voff) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(rsrc)
        : "memory", "m0");
#pragma clang diagnostic pop
}

// 16-byte chunk swizzles.  A kv row occupies 1024 contiguous LDS bytes (64
// chunks); logical chunk c of tile row r lives at physical chunk c ^ sw_kv(r)
// (only the low 4 bits move).  sw_kv is a permutation of 0..15 whose values
// differ in bits [3:2] within every group of 4 consecutive rows and in bits
// [3:1] within every group of 8.  LDS has 64 banks (a 256-byte period); a
// ds_read_b128 serves 16 lanes per pass, four quads of lanes: quad q of a
// half-wave (lanes 4q..4q+3) joins pass parity(popcount(q)).  With the QK
// chunk assignment of each variant and the transposed PV reads, every pass
// touches 16 distinct bank groups (rocprofv3 SQ_LDS_BANK_CONFLICT reads 0).
// A rope row occupies 128 bytes (8 chunks): physical = c ^ sw_rope(r).
__device__ __forceinline__ int sw_kv(int r) {
    return ((r & 3) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);  // uses r mod 16
}
__device__ __forceinline__ int sw_rope(int r) { return (r >> 1) & 7; }

// QK k-order of the specialised-wave and ping-pong kernels: k-step ks (32 of
// the 512 latent dims) takes logical chunks 4 ks .. 4 ks + 3, lane group g
// holding chunk 4 ks + qk_lane_chunk(g), so that one Q fragment load reads a
// whole 64-byte piece of each of its 16 head rows (16 lines per instruction)
// where chunk 16 g + ks reads 16 bytes of 64 lines.  The permutation
// [0, 3, 1, 2] keeps the low two chunk bits of groups 0 and 1 (and of 2 and
// 3) in the same class {0, 3} or {1, 2}, which is what keeps the K reads of
// one ds_read_b128 pass on 16 distinct bank groups under sw_kv (with g in
// place of qk_lane_chunk(g) a pass would meet 2-way conflicts).  Measured:
// C2 -2.4 %, C5 -0.9 %; the column-split kernel (C4 +0.7 % with it) and the
// narrow kernel keep chunk 16 g + ks.
__device__ __forceinline__ int qk_lane_chunk(int g) { return (0x9C >> (2 * g)) & 3; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane reductions over lanes l and l ^ 32 (l ^ 16) with the gfx950
// VALU lane swaps instead of an LDS permute.  v_permlane32_swap on two copies
// of v leaves (v[l], v[l ^ 32]) in the pair on every lane; v_permlane16_swap
// does the same for l ^ 16.
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ------------------------------------------------------------ shared pieces
template <int BN_, int NSTAGE_>
struct Ring {
    static constexpr int BN = BN_;
    static constexpr int NSTAGE = NSTAGE_;
    static constexpr int KV_BYTES = BN * 1024;
    static constexpr int STAGE_BYTES = BN * 1152;
    static constexpr int IDX_OFF = NSTAGE * STAGE_BYTES;
    static constexpr int FLAG_OFF = IDX_OFF + DSA_IDX_CAP * 4;
    static constexpr int LDS_BYTES = FLAG_OFF + 16;
    static constexpr int KV_PER_WAVE = BN / kWaves;        // kv row gathers per wave per tile
    static constexpr int ROPE_PER_WAVE = BN / 8 / kWaves;  // rope gathers (8 rows each)
    static constexpr int LOADS_PER_TILE = KV_PER_WAVE + ROPE_PER_WAVE;  // VMEM ops per wave
    static_assert(BN % (8 * kWaves) == 0, "rope gathers split evenly over the waves");
    static_assert(NSTAGE >= 2 && LOADS_PER_TILE * (NSTAGE - 2) < 64, "vmcnt range");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");

    __device__ static uint32_t stage(uint32_t lds, int t) { return lds + (uint32_t)(t % NSTAGE) * STAGE_BYTES; }

    // Wait until this wave's gathers of tile t have landed, given that the
    // tiles up to min(t + NSTAGE - 2, nt - 1) have been issued (in order).
    __device__ static void wait_tile(int t, int nt) {
        const int ahead = min(NSTAGE - 2, nt - 1 - t);
        if constexpr (NSTAGE >= 4)
            if (ahead >= 2) {
                wait_vmcnt<2 * LOADS_PER_TILE>();
                return;
            }
        if constexpr (NSTAGE >= 3)
            if (ahead >= 1) {
                wait_vmcnt<LOADS_PER_TILE>();
                return;
            }
        wait_vmcnt<0>();
    }
    static_assert(NSTAGE <= 4, "wait_tile handles up to 4 stages");
};

struct WgCoords {
    int token, sp, hgi, b, nt, slot0;
};

// Workgroup -> (row group = token * nsplit + split, head group).  Workgroups
// are dispatched round-robin over the 8 XCDs; when possible all head groups
// of one row group land on the same XCD so the gathered rows are fetched from
// HBM once and re-read from that XCD's L2.
//
// The divisors (head groups, splits, query length) are kernel-uniform and
// nonnegative.  With POW2 (all three powers of two, as on every planned
// benchmark shape) the quotients are shifts and the remainders masks: the
// general division is a dependent chain of a float reciprocal and integer
// corrections (over a hundred instructions for the 64-bit split bounds) that
// sits ahead of the first index load (measured: a 16-head decode workgroup's
// kernel 0.3-0.4 us shorter with shifts).  Both forms give the same values.
template <int BN, bool POW2>
__device__ __forceinline__ WgCoords wg_coords_by(const FwdParams& p) {
    auto quo = [](int a, int d) { return POW2 ? a >> __builtin_ctz(d) : a / d; };
    auto rem = [](int a, int d) { return POW2 ? a & (d - 1) : a % d; };
    auto quo64 = [](int64_t a, int d) { return POW2 ? a >> __builtin_ctz(d) : a / d; };
    const int wg = blockIdx.x;
    int rg, hgi;
    if ((p.rowgroups & 7) == 0) {
        const int j = wg >> 3;
        rg = (wg & 7) + 8 * quo(j, p.hgroups);
        hgi = rem(j, p.hgroups);
    } else {
        rg = quo(wg, p.hgroups);
        hgi = rem(wg, p.hgroups);
    }
    WgCoords c;
    c.token = quo(rg, p.nsplit);
    c.sp = rem(rg, p.nsplit);
    c.hgi = hgi;
    c.b = quo(c.token, p.SQ);
    const int t_begin = (int)quo64((int64_t)c.sp * p.ntiles, p.nsplit);
    const int t_end = (int)quo64((int64_t)(c.sp + 1) * p.ntiles, p.nsplit);
    c.nt = t_end - t_begin;
    c.slot0 = t_begin * BN;
    return c;
}
template <int BN>
__device__ __forceinline__ WgCoords wg_coords(const FwdParams& p) {
    const bool pow2 = ((p.hgroups & (p.hgroups - 1)) | (p.nsplit & (p.nsplit - 1)) | (p.SQ & (p.SQ - 1))) == 0;
    return pow2 ? wg_coords_by<BN, true>(p) : wg_coords_by<BN, false>(p);
}

// Rows of the workgroup's slot range, -1 for every masked slot (including
// the padding of a ragged last tile; nslots <= DSA_IDX_CAP, checked on the
// host).  Split into a global-load half (fetch_indices: the raw loads only,
// nothing waits for them) and a mask-and-store half (store_indices), so the
// caller's Q loads issue while the index loads are in flight (measured: C1's
// main kernel 8.8-8.9 us against 9.0-9.1 us with the wait ahead of Q, C4 -0.9 %;
// the specialised-wave kernel keeps the wait ahead of Q, see there).
template <int CAP = DSA_IDX_CAP>
struct IdxRegs {
    static_assert(CAP % kThreads == 0 && CAP <= DSA_IDX_CAP, "index cache size");
    int v[CAP / kThreads];
};
template <int BN, int CAP = DSA_IDX_CAP>
__device__ __forceinline__ IdxRegs<CAP> fetch_indices(const FwdParams& p, const WgCoords& c) {
    // Buffer loads over the token's index row: a slot past TOPK reads 0
    // (hardware range check) and is then masked.  Being intrinsics rather
    // than plain loads, they are never turned into branches around each load,
    // so all of them issue back to back.
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(p.idx + (int64_t)c.token * p.TOPK), (short)0, p.TOPK * 4, 0x00020000);
    constexpr int N = CAP / kThreads;
    int raw[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
        raw[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (c.slot0 + (int)threadIdx.x + i * kThreads) * 4, 0, 0);
    IdxRegs<CAP> r;
#pragma unroll
    for (int i = 0; i < N; ++i) r.v[i] = raw[i];
    return r;
}
// Every entry of the cache is written (slots past the range hold -1): a
// conditional store would let the compiler sink each global load into its
// branch and wait for it there, serialising the loads.
template <int BN, int CAP>
__device__ __forceinline__ IdxRegs<CAP> mask_indices(const IdxRegs<CAP>& r, const FwdParams& p, const WgCoords& c) {
    // Cached value: the kv row to gather (the pool row when paged), or -1 for
    // a masked slot (index < 0 or >= L, slot past TOPK or past the range).
    constexpr int N = CAP / kThreads;
    const int nslots = c.nt * BN;
    IdxRegs<CAP> res;
    int* out = res.v;
    if (p.block_table == nullptr) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int s = (int)threadIdx.x + i * kThreads;
            const bool ok = (s < nslots) & (c.slot0 + s < p.TOPK) & (r.v[i] >= 0) & (r.v[i] < p.L);
            out[i] = ok ? r.v[i] : -1;
        }
    } else {
        // Second level: the block table row of this batch (again range
        // checked by the buffer descriptor).  An entry outside [0, num_blocks)
        // masks the slot; the test is on the entry itself, so a large entry
        // cannot wrap the 32-bit row product back into the pool.  Inside the
        // pool the row is below num_blocks * block_size < 2^25.
        const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int32_t*>(p.block_table + (int64_t)c.b * p.max_blocks), (short)0, p.max_blocks * 4,
            0x00020000);
        int blk[N];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int id = min(max(r.v[i], 0), p.L - 1);
            blk[i] = __builtin_amdgcn_raw_buffer_load_b32(rb, (id / p.block_size) * 4, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int s = (int)threadIdx.x + i * kThreads;
            const int id = min(max(r.v[i], 0), p.L - 1);
            const bool in_pool = (uint32_t)blk[i] < (uint32_t)p.num_blocks;
            const int row = (in_pool ? blk[i] : 0) * p.block_size + id % p.block_size;
            const bool ok = (s < nslots) & (c.slot0 + s < p.TOPK) & (r.v[i] >= 0) & (r.v[i] < p.L) & in_pool;
            out[i] = ok ? row : -1;
        }
    }
    return res;
}
template <int BN, int CAP>
__device__ __forceinline__ void store_indices(const IdxRegs<CAP>& r, uint32_t idx_lds, const FwdParams& p,
                                              const WgCoords& c) {
    const IdxRegs<CAP> m = mask_indices<BN>(r, p, c);
#pragma unroll
    for (int i = 0; i < CAP / kThreads; ++i)
        lds_store<int>(idx_lds + 4 * ((int)threadIdx.x + i * kThreads), m.v[i]);
}

// Compaction of the workgroup's slots (threads 0..255 hold the masked cache
// values of mask_indices): the valid entries, in slot order, go to the front
// of the cache and the last tile is padded with -1, so masked slots cost no
// gather and no MFMA work.  A masked slot contributes exactly nothing (its
// score is -inf), so the result changes only by the order of the FP32 sums.
// Two halves around a workgroup barrier that every wave passes:
// compact_count (threads 0..255: each wave publishes the valid count of each
// of its N chunks to `counts`, 4 N ints of LDS) and, after the barrier,
// compact_store (threads 0..255: entries to their ranks, padding) and
// compact_total (every thread: the valid count, for the tile count).
template <int CAP>
__device__ __forceinline__ void compact_count(const IdxRegs<CAP>& m, uint32_t counts) {
    constexpr int N = CAP / kThreads;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const uint64_t b = __ballot(m.v[i] >= 0);
        if (lane == i) lds_store<int>(counts + 4 * (w * N + i), __popcll(b));
    }
}
template <int CAP>
__device__ __forceinline__ int compact_total(uint32_t counts) {
    constexpr int N = CAP / kThreads;
    int total = 0;
#pragma unroll
    for (int k = 0; k < 4 * N; k += 4) {
        const i32x4 v = lds_load<i32x4>(counts + 4 * k);
        total += v[0] + v[1] + v[2] + v[3];
    }
    return total;
}
template <int BN, int CAP>
__device__ __forceinline__ void compact_store(const IdxRegs<CAP>& m, uint32_t counts, uint32_t idx_lds, int total) {
    constexpr int N = CAP / kThreads;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int base = 0;  // valid entries of the earlier chunks
#pragma unroll
    for (int i = 0; i < N; ++i) {
        int before = 0, all = 0;  // this chunk: in earlier waves, in every wave
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const int n = lds_load<int>(counts + 4 * (ww * N + i));
            before += ww < w ? n : 0;
            all += n;
        }
        const uint64_t b = __ballot(m.v[i] >= 0);
        const int rank = base + before +
                         (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        if (m.v[i] >= 0) lds_store<int>(idx_lds + 4 * rank, m.v[i]);
        base += all;
    }
    const int pad = total + (int)threadIdx.x;
    if ((int)threadIdx.x < BN && pad < (total + BN - 1) / BN * BN) lds_store<int>(idx_lds + 4 * pad, -1);
}

// Buffer resources over this workgroup's batch of kv and k_rope.
struct Gather {
    const char* kv;  // first kv row of the addressed range
    rsrc_t kr;       // k_rope rows of the range (32-bit per-lane offsets: < 2^25 rows)
};
__device__ __forceinline__ Gather make_gather(const FwdParams& p, int b) {
    const int64_t rows = p.block_table ? 0 : (int64_t)b * p.L;  // first row of the addressed range
    Gather g;
    g.kv = reinterpret_cast<const char*>(p.kv) + rows * 1024;
    g.kr = make_rsrc(reinterpret_cast<const char*>(p.k_rope) + rows * 128, (uint32_t)p.kv_rows * 128u);
    return g;
}

// Gather of workgroup tile t into ring stage `stage` (LDS byte address).
// Wave w fetches kv rows [w*KV_PER_WAVE, (w+1)*KV_PER_WAVE) (1 KiB each, one
// instruction per row) and ROPE_PER_WAVE groups of 8 rope rows.  A masked
// slot (-1 in the index cache) gathers row 0; its score is masked later.
template <class R>
__device__ __forceinline__ void issue_tile(const FwdParams& p, const Gather& gt, int t, uint32_t stage,
                                           uint32_t idx_lds, int wave, int lane) {
    const int rows = p.kv_rows;
    const int r0 = wave * R::KV_PER_WAVE;
    const int my_id = lds_load<int>(idx_lds + 4 * (t * R::BN + r0 + (lane % R::KV_PER_WAVE)));
    const uint32_t my_row = (uint32_t)min(max(my_id, 0), rows - 1);
    const uint32_t lane16 = (uint32_t)lane << 4;
#pragma unroll
    for (int rr = 0; rr < R::KV_PER_WAVE; ++rr) {
        const int r = r0 + rr;
        gather_row(stage + r * 1024, row_rsrc(gt.kv, __builtin_amdgcn_readlane(my_row, rr)), lane16,
                   (uint32_t)sw_kv(r) << 4);
    }
#pragma unroll
    for (int jj = 0; jj < R::ROPE_PER_WAVE; ++jj) {
        const int j = wave * R::ROPE_PER_WAVE + jj;
        const int r = j * 8 + (lane >> 3);
        const int id = lds_load<int>(idx_lds + 4 * (t * R::BN + r));
        const uint32_t voff = ((uint32_t)min(max(id, 0), rows - 1) << 7) + (((lane & 7) ^ sw_rope(r)) << 4);
        gather_lanes(stage + R::KV_BYTES + j * 1024, gt.kr, voff);
    }
}

// Store 4 consecutive bf16 outputs of one head row.
__device__ __forceinline__ void store_bf16x4(uint16_t* dst, float a, float b, float c, float d) {
    bf16x4 v;
    v[0] = (__bf16)a;
    v[1] = (__bf16)b;
    v[2] = (__bf16)c;
    v[3] = (__bf16)d;
    *reinterpret_cast<bf16x4*>(dst) = v;
}

// ====================================================================== wide
// HW head-waves of 32 heads x KW kv-waves (HW * KW == 4); every wave processes
// one 32-row subtile of each BN-row tile (BN == 32 * KW): wave (hw, kw) owns
// rows [32*kw, 32*kw + 32) for heads hw*32..+31.
//
// 32x32x16 operand layouts (lane i, h = i >> 5, n = i & 31):
//   A[m = n][k = 8h + j], B[k = 8h + j][n = n], C[m = 8*(r>>2) + 4h + (r&3)][n = n].
template <int HW, int KW, int BN, int NSTAGE>
__global__ __launch_bounds__(kThreads, 1) void sparse_mla_fwd_wide(FwdParams p) {
    using R = Ring<BN, NSTAGE>;
    static_assert(HW * KW == kWaves && BN == 32 * KW, "wide variant shape");
    __shared__ __attribute__((aligned(1024))) char smem[R::LDS_BYTES];
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hw = wave % HW;
    const int kw = wave / HW;
    const int h = lane >> 5;
    const int n32 = lane & 31;

    const WgCoords c = wg_coords<BN>(p);
    const int head = c.hgi * (32 * HW) + hw * 32 + n32;  // this lane's head
    const uint32_t idx_lds = lds + R::IDX_OFF;

    // Index loads first: the first gather depends on them, Q only on the
    // first MFMA.
    const IdxRegs<> ids = fetch_indices<BN>(p, c);

    // ---- Q fragments: B operand of S^T = K . Q^T.  Lane holds
    // Q[head][16*ks + 8*h .. +7]; ks 32..35 come from q_rope.
    bf16x8 qf[36];
    {
        const uint16_t* qrow = p.q + ((int64_t)c.token * p.H + head) * 512 + 8 * h;
#pragma unroll
        for (int ks = 0; ks < 32; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + 16 * ks);
        const uint16_t* rrow = p.q_rope + ((int64_t)c.token * p.H + head) * 64 + 8 * h;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[32 + ks] = *reinterpret_cast<const bf16x8*>(rrow + 16 * ks);
    }
    store_indices<BN>(ids, idx_lds, p, c);
    lds_barrier();
    const Gather gt = make_gather(p, c.b);

    const int row0 = kw * 32;

    // ---- running state (log2 units)
    f32x16 oacc[16];
    float m_ref = -FLT_MAX;   // reference max of P
    float m_true = -FLT_MAX;  // exact running max
    float l_run = 0.f;        // per-lane partial of the head's sum, relative to m_ref
    const uint32_t flag_lds = lds + R::FLAG_OFF;

    // At most two passes over the range (see kRestartLog2).  Pass 0 fixes
    // m_ref at the first tile with a valid row; if any head's max later grows
    // past m_ref + kRestartLog2, pass 1 recomputes the range with m_ref = the
    // exact max found by pass 0, which no score can exceed.
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[i] = f32x16{};
        l_run = 0.f;
        if (pass == 1) m_ref = m_true;
        bool overflow = false;
#pragma unroll
        for (int i = 0; i < NSTAGE - 1; ++i)
            if (i < c.nt) issue_tile<R>(p, gt, i, R::stage(lds, i), idx_lds, wave, lane);
        // The Q loads complete here, with the first tiles.  The compiler does
        // not count the gathers (inline asm), so a wait it placed for Q inside
        // the loop would be a vmcnt(0) on every tile, draining the ring.
        wait_vmcnt<0>();

        for (int t = 0; t < c.nt; ++t) {
            R::wait_tile(t, c.nt);
            lds_barrier();  // tile t visible to all waves; stage of tile t-1 free
            if (t + NSTAGE - 1 < c.nt)
                issue_tile<R>(p, gt, t + NSTAGE - 1, R::stage(lds, t + NSTAGE - 1), idx_lds, wave, lane);
            const uint32_t stage = R::stage(lds, t);
            // Per-lane fragment offsets, recomputed every tile from a lane id
            // the compiler cannot see through (keeps ~20 VGPRs free across the
            // loop instead of hoisting these invariants and spilling).
            // Swizzles depend on the row mod 16 and XOR only the low 4 bits of
            // a chunk index, so each fragment address is one of these bases
            // plus a compile-time multiple of 256 bytes.
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int lh = ln >> 5, ln32 = ln & 31, lG = ln >> 4, ln16 = ln & 15;
            const int ltr = 4 * lh + (ln16 >> 2);

            // ---- S^T = K . Q^T for rows row0..row0+31: one MFMA chain (32x32
            // accumulation chains issue back to back) in an explicit 4-deep LDS
            // pipeline; the scheduler is fenced per step so at most 4 fragments
            // are live.
            f32x16 sacc = f32x16{};
            // Slot indices of this lane's 16 score rows (for the mask), read
            // before the MFMAs so their LDS latency is hidden.
            i32x4 ivs[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) ivs[q] = lds_load<i32x4>(idx_lds + 4 * (t * BN + row0 + 8 * q + 4 * lh));
            const uint32_t rowa = stage + (row0 + ln32) * 1024;
            const uint32_t rowr = stage + R::KV_BYTES + (row0 + ln32) * 128;
            // QK A operand: row row0 + n32, logical chunk 2*ks + h = 16*(ks >> 3) + (2*(ks & 7) + h)
            uint32_t qa[8], ra[4];
#pragma unroll
            for (int j = 0; j < 8; ++j) qa[j] = rowa + (((2 * j + lh) ^ sw_kv(ln32)) << 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) ra[j] = rowr + (((2 * j + lh) ^ sw_rope(ln32 & 15)) << 4);
            auto kfrag = [&](int ks) -> bf16x8 {
                return ks < 32 ? lds_load<bf16x8>(qa[ks & 7] + ((ks >> 3) << 8)) : lds_load<bf16x8>(ra[ks - 32]);
            };
            bf16x8 kf[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) kf[j] = kfrag(j);
#pragma unroll
            for (int ks = 0; ks < 36; ++ks) {
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks & 3], qf[ks], sacc, 0, 0, 0);
                if (ks + 4 < 36) kf[ks & 3] = kfrag(ks + 4);
                __builtin_amdgcn_sched_barrier(0);
            }

            // ---- scale, mask, online softmax.  Lane holds rows
            // row0 + 8*q + 4*h + (0..3) for q = 0..3 (register 4q + j) of head n32.
            // Raw scores with masked rows at -inf; the scale folds into the max
            // (positive factor: max(c*s) = c*max(s)) and into one FMA per
            // score for P = exp2(c*s - m_ref).
            float x[16];
            float smax = -INFINITY;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool valid = ivs[q][j] >= 0;
                    x[4 * q + j] = valid ? sacc[4 * q + j] : -INFINITY;
                    smax = fmaxf(smax, x[4 * q + j]);
                }
            }
            smax = max_xor32(smax);
            m_true = fmaxf(m_true, smax * p.score_scale_log2);
            if (m_ref == -FLT_MAX) m_ref = m_true;  // first valid rows: O and l are still zero
            const bool ovf = m_true > m_ref + kRestartLog2;
            overflow |= ovf;
            const float neg_ref = -m_ref;
            bf16x8 pk[2];
            float psum = 0.f;
            if (__any(ovf)) {
                // This pass is to be discarded; the clamp keeps it free of inf.
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e = fast_exp2(fminf(fmaf(x[r], p.score_scale_log2, neg_ref), kRestartLog2));
                    psum += e;
                    pk[r >> 3][r & 7] = (__bf16)e;
                }
            } else {  // every P <= 2^kRestartLog2
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e = fast_exp2(fmaf(x[r], p.score_scale_log2, neg_ref));
                    psum += e;
                    pk[r >> 3][r & 7] = (__bf16)e;
                }
            }
            l_run += psum;

            // ---- O^T += V^T . P^T, two k-steps of 16 rows x 16 column blocks,
            // same 4-deep pipeline over the 32 (kk, cb) steps.
            // PV A operand (transposed reads): for k-step kk and read rd, row
            // row0 + 16*kk + 8*rd + 4*h + n16/4, columns 32*cb + 16*(G&1) + 4*(n16&3)
            // -> logical chunk 4*cb + 2*(G&1) + ((n16&3)>>1) = 16*(cb >> 2) + (4*(cb&3) + ...),
            // byte 8*(n16&1) within the chunk.
            const uint32_t vrow = stage + (row0 + ltr) * 1024;
            uint32_t va[2][4];
#pragma unroll
            for (int rd = 0; rd < 2; ++rd)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    va[rd][j] = vrow + rd * 8 * 1024 +
                                (((4 * j + 2 * (lG & 1) + ((ln16 & 3) >> 1)) ^ sw_kv(ltr + 8 * rd)) << 4) +
                                ((ln16 & 1) << 3);
            auto vfrag = [&](int step) -> bf16x8 {
                const int kk = step >> 4, cb = step & 15;
                const uint32_t imm = kk * 16 * 1024 + ((cb >> 2) << 8);
                const bf16x4 v0 = lds_load_tr(va[0][cb & 3] + imm);
                const bf16x4 v1 = lds_load_tr(va[1][cb & 3] + imm);
                return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
            };
            bf16x8 vf[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) vf[j] = vfrag(j);
#pragma unroll
            for (int step = 0; step < 32; ++step) {
                const int kk = step >> 4, cb = step & 15;
                oacc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[step & 3], pk[kk], oacc[cb], 0, 0, 0);
                if (step + 4 < 32) vf[step & 3] = vfrag(step + 4);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // ---- workgroup vote: does any head need pass 1?
        if (pass == 1) break;
        if (threadIdx.x == 0) lds_store<int>(flag_lds, 0);
        lds_barrier();  // also: every wave is past its last ring read
        if (__any(overflow) && lane == 0) lds_store<int>(flag_lds, 1);
        lds_barrier();
        if (__builtin_amdgcn_readfirstlane(lds_load<int>(flag_lds)) == 0) break;
    }

    // ---- epilogue.  Lane-derived values are recomputed from an opaque lane
    // id: kept live from the prologue they would be spilled, and each reload
    // waits (vmcnt(0)) for every output store already issued.
    l_run = sum_xor32(l_run);
    int eln = lane;
    asm volatile("" : "+v"(eln));
    const int eh = eln >> 5, en32 = eln & 31;
    const int ehead = c.hgi * (32 * HW) + hw * 32 + en32;
    if constexpr (KW == 2) {
        // kv-wave 1 hands (m_ref, m_true, l, O) to kv-wave 0 of the same head
        // slice through LDS; kv-wave 0 merges (m = max, w = exp(m_k - m)).
        constexpr int OX_STRIDE = 516;  // floats per head row, padded
        static_assert(HW * 32 * OX_STRIDE * 4 <= R::IDX_OFF, "exchange fits the ring");
        lds_barrier();                  // every wave is past its last ring read
        const uint32_t ml = lds + R::IDX_OFF;
        const uint32_t ox = lds + ((hw * 32 + en32) * OX_STRIDE + 4 * eh) * 4;
        if (kw == 1) {
            if (eh == 0) {
                lds_store<float>(ml + 4 * (hw * 32 + en32), m_ref);
                lds_store<float>(ml + 4 * (64 + hw * 32 + en32), m_true);
                lds_store<float>(ml + 4 * (128 + hw * 32 + en32), l_run);
            }
#pragma unroll
            for (int cb = 0; cb < 16; ++cb)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    lds_store<f32x4>(ox + (32 * cb + 8 * q) * 4,
                                     f32x4{oacc[cb][4 * q], oacc[cb][4 * q + 1], oacc[cb][4 * q + 2],
                                           oacc[cb][4 * q + 3]});
        }
        lds_barrier();
        if (kw == 1) return;
        const float m1 = lds_load<float>(ml + 4 * (hw * 32 + en32));
        const float t1 = lds_load<float>(ml + 4 * (64 + hw * 32 + en32));
        const float l1 = lds_load<float>(ml + 4 * (128 + hw * 32 + en32));
        const float mm = fmaxf(m_ref, m1);
        const float w0 = fast_exp2(m_ref - mm), w1 = fast_exp2(m1 - mm);
        l_run = w0 * l_run + w1 * l1;
        m_ref = mm;
        m_true = fmaxf(m_true, t1);
#pragma unroll
        for (int cb = 0; cb < 16; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = lds_load<f32x4>(ox + (32 * cb + 8 * q) * 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) oacc[cb][4 * q + j] = w0 * oacc[cb][4 * q + j] + w1 * v[j];
            }
    }

    // Re-express (m_ref, l, O) against the true max for the caller.
    const float to_true = fast_exp2(m_ref - m_true);
    const float l_fin = l_run * to_true;
    const float m_nat = m_true * kLn2;
    if (p.nsplit == 1 && KW == 1) {
        // The bf16 rows of all 32 * HW heads go through the (now idle) ring
        // first, so that every global store instruction writes one head's
        // whole 1 KiB row: a lane holds 4 columns of each of 16 column blocks
        // of one head, a scattered 8-byte pattern in memory.
        constexpr int HROW = 1040;  // bytes per staged head row (1 KiB + 16: spreads heads over the banks)
        static_assert(HW * 32 * HROW <= R::IDX_OFF, "staged rows fit the ring");
        const float inv_l = 1.0f / l_run;  // O and l_run share m_ref
        lds_barrier();                     // every wave is past its last ring read
        const uint32_t srow = lds + (uint32_t)((hw * 32 + en32) * HROW + 8 * eh);
#pragma unroll
        for (int cb = 0; cb < 16; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                bf16x4 v;
                v[0] = (__bf16)(oacc[cb][4 * q] * inv_l);
                v[1] = (__bf16)(oacc[cb][4 * q + 1] * inv_l);
                v[2] = (__bf16)(oacc[cb][4 * q + 2] * inv_l);
                v[3] = (__bf16)(oacc[cb][4 * q + 3] * inv_l);
                lds_store<bf16x4>(srow + 2 * (32 * cb + 8 * q), v);
            }
        if (eh == 0) {
            p.out_max[(int64_t)c.token * p.H + ehead] = m_nat;
            p.out_sum[(int64_t)c.token * p.H + ehead] = l_fin;
        }
        lds_barrier();
        // wave w stores head rows w, w + 4, ...: 64 lanes x 16 bytes = one row
        uint16_t* obase = p.out + ((int64_t)c.token * p.H + c.hgi * (32 * HW)) * 512 + 8 * eln;
#pragma unroll 4
        for (int hr = wave; hr < HW * 32; hr += kWaves)
            *reinterpret_cast<bf16x8*>(obase + (int64_t)hr * 512) = lds_load<bf16x8>(lds + hr * HROW + 16 * eln);
    } else if (p.nsplit == 1) {
        const float inv_l = 1.0f / l_run;  // O and l_run share m_ref
        uint16_t* orow = p.out + ((int64_t)c.token * p.H + ehead) * 512 + 4 * eh;
#pragma unroll
        for (int cb = 0; cb < 16; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                store_bf16x4(orow + 32 * cb + 8 * q, oacc[cb][4 * q] * inv_l, oacc[cb][4 * q + 1] * inv_l,
                             oacc[cb][4 * q + 2] * inv_l, oacc[cb][4 * q + 3] * inv_l);
        if (eh == 0) {
            p.out_max[(int64_t)c.token * p.H + ehead] = m_nat;
            p.out_sum[(int64_t)c.token * p.H + ehead] = l_fin;
        }
    } else {
        const int64_t prow = ((int64_t)c.token * p.nsplit + c.sp) * p.H + ehead;
        float* orow = p.part_o + prow * 512 + 4 * eh;
#pragma unroll
        for (int cb = 0; cb < 16; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<f32x4*>(orow + 32 * cb + 8 * q) =
                    f32x4{oacc[cb][4 * q], oacc[cb][4 * q + 1], oacc[cb][4 * q + 2], oacc[cb][4 * q + 3]} *
                    to_true;
        if (eh == 0) {
            p.part_m[prow] = m_nat;
            p.part_l[prow] = l_fin;
        }
    }
}

// ============================================================ fp8 kv rows
// FP8 KV cache row (656 bytes per token, the layout of DeepSeek-V3.2's FP8
// MLA cache): 512 OCP float8 e4m3 latent values, 4 fp32 scales (scale i
// covers dims 128 i .. 128 i + 127), then the 64 bf16 rope values.  A tile's
// rows land as stored (656-byte stride) in one of two raw LDS stages; every
// wave then expands a quarter of the latent dims of all its rows,
//   kv[d] = bf16(fp32(e4m3[d]) * scale[d / 128])      (both roundings RNE),
// into one bf16 tile laid out and swizzled like Ring's kv region, so the MFMA
// code reads it unchanged.  Rope values are read from the raw rows.
constexpr int kFp8Row = 656;
constexpr int kFp8ScaleOff = 512;
constexpr int kFp8RopeOff = 528;

template <int BN_>
struct RingFp8 {
    static constexpr int BN = BN_;
    static constexpr int NSTAGE = 2;
    static constexpr int RAW_BYTES = BN * kFp8Row;       // one raw stage
    static constexpr int KV_OFF = NSTAGE * RAW_BYTES;     // bf16 latent tile [BN][1024]
    static constexpr int IDX_OFF = KV_OFF + BN * 1024;
    static constexpr int FLAG_OFF = IDX_OFF + DSA_IDX_CAP * 4;
    static constexpr int LDS_BYTES = FLAG_OFF + 16;
    static constexpr int KV_PER_WAVE = BN / kWaves;  // one load per row, rope included
    static constexpr int LOADS_PER_TILE = KV_PER_WAVE;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(RAW_BYTES % 16 == 0, "16-byte aligned stages");
    __device__ static uint32_t raw(uint32_t lds, int t) { return lds + (uint32_t)(t % NSTAGE) * RAW_BYTES; }
};

// The kv cache (or pool) as bytes, from the first row of the addressed range.
__device__ __forceinline__ const char* fp8_base(const FwdParams& p, int b) {
    const int64_t rows = p.block_table ? 0 : (int64_t)b * p.L;
    return reinterpret_cast<const char*>(p.kv) + rows * kFp8Row;
}

// One fp8 row through a descriptor at its 64-bit address with a 656-byte
// range; lanes 0..40 each load 16 bytes to m0 + 16 * lane (the other lanes
// are masked off, so nothing lands past the row).
__device__ __forceinline__ rsrc_t fp8_row_rsrc(const char* base, uint32_t row) {
    const uint64_t a = reinterpret_cast<uint64_t>(base) + (uint64_t)row * kFp8Row;
    rsrc_t r;
    r[0] = (int)(uint32_t)a;
    r[1] = (int)((a >> 32) & 0xffff);
    r[2] = kFp8Row;
    r[3] = 0x00020000;
    return r;
}

template <class R>
__device__ __forceinline__ void issue_tile_fp8(const FwdParams& p, const char* base, int t, uint32_t raw_stage,
                                               uint32_t idx_lds, int wave, int lane) {
    const int rows = p.kv_rows;
    const int r0 = wave * R::KV_PER_WAVE;
    const int my_id = lds_load<int>(idx_lds + 4 * (t * R::BN + r0 + (lane % R::KV_PER_WAVE)));
    const uint32_t my_row = (uint32_t)min(max(my_id, 0), rows - 1);
    const uint32_t voff = (uint32_t)lane << 4;
#pragma unroll
    for (int rr = 0; rr < R::KV_PER_WAVE; ++rr) {
        const rsrc_t rs = fp8_row_rsrc(base, __builtin_amdgcn_readlane(my_row, rr));
        if (lane < kFp8Row / 16) gather_lanes(raw_stage + (r0 + rr) * kFp8Row, rs, voff);
    }
}

// One lane's 128 latent values (16-byte chunks 16 b .. 16 b + 15 of its row,
// raw bytes at src, scale sc) into the swizzled bf16 row at dst.
__device__ __forceinline__ void expand_block(uint32_t src, float sc, uint32_t dst, uint32_t sw, uint32_t b) {
    i32x4 v[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) v[m] = lds_load<i32x4>(src + 16 * m);
    // A power-of-two scale 2^k (k in [-100, 100]) makes fp32(e4m3) * scale
    // exact in fp32 and in bf16, and v_cvt_scalef32_pk_bf16_fp8 -- which
    // applies only the exponent of its scale -- then yields the same bits in
    // one instruction per two values.  The branch is uniform per wave.
    const uint32_t sb = __float_as_uint(sc);
    const uint32_t sexp = (sb >> 23) & 0xffu;
    const bool pow2 = (sb & 0x807fffffu) == 0 && sexp >= 27u && sexp <= 227u;
    auto store = [&](int m, int h, const bf16x8& o) {
        const uint32_t chunk = 16u * b + (uint32_t)(2 * m + h);  // logical: dims 8 chunk ..
        lds_store<bf16x8>(dst + ((chunk ^ sw) << 4), o);
    };
    if (__all(pow2)) {
#pragma unroll
        for (int m = 0; m < 8; ++m) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                bf16x8 o;
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const int w = v[m][2 * h + d];
                    const auto lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, sc, false);
                    const auto hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, sc, true);
                    o[4 * d + 0] = lo[0];
                    o[4 * d + 1] = lo[1];
                    o[4 * d + 2] = hi[0];
                    o[4 * d + 3] = hi[1];
                }
                store(m, h, o);
            }
        }
    } else {
#pragma unroll
        for (int m = 0; m < 8; ++m) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // 8 values = one 16-byte bf16 chunk
                bf16x8 o;
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const int w = v[m][2 * h + d];
                    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
                    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
                    o[4 * d + 0] = (__bf16)(lo[0] * sc);
                    o[4 * d + 1] = (__bf16)(lo[1] * sc);
                    o[4 * d + 2] = (__bf16)(hi[0] * sc);
                    o[4 * d + 3] = (__bf16)(hi[1] * sc);
                }
                store(m, h, o);
            }
        }
    }
}

// Tile-wide expansion (head slices share rows): wave w expands dims
// 128 w .. 128 w + 127 of every row; lane l takes row l.  Reads at a 656-byte
// stride hit 16 distinct bank groups per pass, and so do the swizzled writes.
template <class R>
__device__ __forceinline__ void dequant_tile(uint32_t raw_stage, uint32_t kv_tile, int wave, int lane) {
    static_assert(R::BN == 64, "one row per lane");
    const uint32_t row = (uint32_t)lane;
    expand_block(raw_stage + row * kFp8Row + 128u * (uint32_t)wave,
                 lds_load<float>(raw_stage + row * kFp8Row + kFp8ScaleOff + 4u * (uint32_t)wave),
                 kv_tile + row * 1024u, (uint32_t)sw_kv(lane), (uint32_t)wave);
}

// Per-wave expansion of the 16 rows a wave alone reads (one head slice): lane
// l takes row rowbase + l % 16 and block 2 ((l / 16) % 2) + l / 32.  A pass
// serves lanes 16 l / 16 .. (k-groups 0 and 1, or 2 and 3), i.e. blocks 0 and
// 2 (or 1 and 3), 256 bytes apart -- the same bank groups -- over
// complementary sets of 8 rows, which the 656-byte row stride (9 r mod 16 in
// 16-byte groups) spreads over all 16 bank groups.
__device__ __forceinline__ void dequant_rows(uint32_t raw_stage, uint32_t kv_tile, int rowbase, int lane) {
    const uint32_t row = (uint32_t)(rowbase + (lane & 15));
    const uint32_t b = 2u * (uint32_t)((lane >> 4) & 1) + (uint32_t)(lane >> 5);
    expand_block(raw_stage + row * kFp8Row + 128u * b,
                 lds_load<float>(raw_stage + row * kFp8Row + kFp8ScaleOff + 4u * b),
                 kv_tile + row * 1024u, (uint32_t)sw_kv((int)row), b);
}

// ==================================================================== narrow
// HW head-waves of 16 heads x KW kv-waves (HW * KW == 4).
//
// 16x16x32 operand layouts (lane i, g = i >> 4, n = i & 15):
//   A[m = n][k = 8g + j], B[k = 8g + j][n = n], C[m = 4g + r][n = n].
// ---------------------------------------------------- in-kernel split merge
// With p.arrivals set, every workgroup of a (token, head group) stores its
// split partials with agent-coherent accesses (the cache policy of an
// agent-scope atomic: sc1, written through to the level every XCD reads),
// waits for them to complete, and counts itself in on the group's arrival
// counter with an agent-scope atomic; the workgroup that arrives last reads
// all the group's partials back with agent-coherent loads, merges them with
// merge_math.h -- the merge kernel's arithmetic, so the bits are the same --
// writes out, out_max and out_sum, and zeroes the counter for the next call.
// Because every access to the partials is coherent at agent scope, no L2
// writeback or invalidation (an agent-scope fence) is needed.  No workgroup
// waits for another, so nothing depends on which workgroups are resident.
//
// A lane owns head `head` = head0 + hl and columns 16 cb + 4 g .. +3 for cb
// in [cb_lo, cb_lo + NCB); its partials of split s live in the group's
// head block of that split: part_o row (token * nsplit + s) * H + head0,
// byte 2048 hl + 16 g + 64 cb.
constexpr int kAgentCoherent = 16;  // buffer cache policy: sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t group_block(const FwdParams& p, int token, int split, int head0,
                                                              int heads) {
    return __builtin_amdgcn_make_buffer_rsrc(p.part_o + (((int64_t)token * p.nsplit + split) * p.H + head0) * 512,
                                             (short)0, heads * 2048, 0x00020000);
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// FP32 partial rows staged in LDS: row hl of the workgroup's heads at
// stage + kPartRow * hl (the 16 extra bytes put the 16 rows that one
// ds_write_b128 pass touches on distinct banks).
//
// A lane's accumulators hold 4 columns of one head per column block, so a
// store straight from them writes sixteen 64-byte pieces of 16 head rows per
// instruction, and the cost of the partial stores tracks those pieces, not
// the bytes.  Staged in the (then free) ring and stored as whole 1 KiB
// halves of a row, each instruction writes 8 full 128-byte lines: main
// kernel C2 -0.8 us, C1 -0.4 us, C3 -1.3 us, outputs bit-identical.
constexpr int kPartRow = 2048 + 16;
enum PartStore { kPartPlain = 0, kPartNonTemporal = 1, kPartAgent = 2 };

// Store of the workgroup's `heads` staged partial rows to part_o as whole
// 1 KiB halves of a row (one instruction each), wave w of nwaves taking
// halves w, w + nwaves, ...  Non-temporal for the partials only the merge
// kernel reads (the specialised-wave kernel's: -0.8 us at C2 against plain
// stores; level for the column-split kernel's), agent-coherent for the
// in-kernel merge.
template <int MODE>
__device__ __forceinline__ void store_staged_partials(const FwdParams& p, const WgCoords& c, int head0, int heads,
                                                      uint32_t stage, int wave, int nwaves, int lane) {
    if constexpr (MODE == kPartAgent) {
        const __amdgpu_buffer_rsrc_t rs = group_block(p, c.token, c.sp, head0, heads);
        for (int i = wave; i < 2 * heads; i += nwaves) {
            const u32x4 v = lds_load<u32x4>(stage + (uint32_t)((i >> 1) * kPartRow + 1024 * (i & 1) + 16 * lane));
            __builtin_amdgcn_raw_buffer_store_b128(v, rs, (i >> 1) * 2048 + 1024 * (i & 1) + 16 * lane, 0,
                                                   kAgentCoherent);
        }
    } else {
        float* base = p.part_o + (((int64_t)c.token * p.nsplit + c.sp) * p.H + head0) * 512 + 4 * lane;
        for (int i = wave; i < 2 * heads; i += nwaves) {
            const f32x4 v = lds_load<f32x4>(stage + (uint32_t)((i >> 1) * kPartRow + 1024 * (i & 1) + 16 * lane));
            f32x4* dst = reinterpret_cast<f32x4*>(base + (i >> 1) * 512 + 256 * (i & 1));
            if constexpr (MODE == kPartNonTemporal)
                __builtin_nontemporal_store(v, dst);
            else
                *dst = v;
        }
    }
}

// Count-in of a workgroup's partials (every wave calls it): true in the
// workgroup that arrives last, which then owns the group's merge and has
// zeroed the counter for the next call.
__device__ __forceinline__ bool group_count_in(const FwdParams& p, const WgCoords& c, uint32_t flag_lds) {
    wait_vmcnt<0>();  // this wave's partial stores have completed ...
    lds_barrier();    // ... and every other wave's
    const int64_t group = (int64_t)c.token * p.hgroups + c.hgi;
    if (threadIdx.x == 0) {
        const uint32_t before =
            __hip_atomic_fetch_add(p.arrivals + group, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds_store<int>(flag_lds, before + 1 == (uint32_t)p.nsplit ? 1 : 0);
    }
    lds_barrier();
    if (__builtin_amdgcn_readfirstlane(lds_load<int>(flag_lds)) == 0) return false;
    if (threadIdx.x == 0) __hip_atomic_store(p.arrivals + group, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// The merge of a group by its last workgroup: this lane's columns, SPR
// splits' partials in flight per round trip (the sum runs over the splits in
// ascending order whatever SPR is).
template <int NCB, int SPR = 4>
__device__ __forceinline__ void merge_group_cols(const FwdParams& p, const WgCoords& c, int head0, int heads, int hl,
                                                 int g, bool writes_ml, int cb_lo) {
    static_assert(NCB % 8 == 0, "column blocks per lane");
    const int S = p.nsplit;  // 2..16, checked on the host
    const int head = head0 + hl;
    const int64_t row0 = (int64_t)c.token * S * p.H + head;  // (m, l) of split s: row0 + s * H
    float ms[16], ls[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        ms[s] = s < S ? __hip_atomic_load(p.part_m + row0 + (int64_t)s * p.H, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT)
                      : -FLT_MAX;
        ls[s] = s < S ? __hip_atomic_load(p.part_l + row0 + (int64_t)s * p.H, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT)
                      : 0.f;
    }
    float m = -FLT_MAX;
#pragma unroll
    for (int s = 0; s < 16; ++s) m = fmaxf(m, ms[s]);
    float w[16];
    float l = 0.f;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        w[s] = merge_weight(ms[s], m);
        if (s < S) l = __builtin_fmaf(w[s], ls[s], l);
    }
    const uint32_t voff = (uint32_t)(hl * 2048 + 16 * g + 64 * cb_lo);
    uint16_t* orow = p.out + ((int64_t)c.token * p.H + head) * 512 + 4 * g + 16 * cb_lo;
#pragma unroll
    for (int c8 = 0; c8 < NCB; c8 += 8) {
        merge_f32x4 acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = merge_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s0 = 0; s0 < 16; s0 += SPR) {
            if (s0 < S) {
                merge_f32x4 u[SPR][8];
#pragma unroll
                for (int j = 0; j < SPR; ++j) {
                    if (s0 + j < S) {
                        const __amdgpu_buffer_rsrc_t rs = group_block(p, c.token, s0 + j, head0, heads);
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            u[j][i] = __builtin_bit_cast(
                                merge_f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 64 * (c8 + i), 0,
                                                                                   kAgentCoherent));
                    }
                }
#pragma unroll
                for (int j = 0; j < SPR; ++j)
                    if (s0 + j < S)
#pragma unroll
                        for (int i = 0; i < 8; ++i) merge_add_cols(w[s0 + j], u[j][i], acc[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<merge_bf16x4*>(orow + 16 * (c8 + i)) = merge_finish(acc[i], l);
    }
    if (writes_ml) {
        p.out_max[(int64_t)c.token * p.H + head] = m;
        p.out_sum[(int64_t)c.token * p.H + head] = l;
    }
}

template <int NCB>
__device__ __forceinline__ void merge_if_last(const FwdParams& p, const WgCoords& c, int head0, int heads, int hl,
                                              int g, bool writes_ml, int cb_lo, uint32_t flag_lds) {
    if (group_count_in(p, c, flag_lds)) merge_group_cols<NCB>(p, c, head0, heads, hl, g, writes_ml, cb_lo);
}

template <int HW, int KW, bool FP8 = false>
__global__ __launch_bounds__(kThreads, 1) void sparse_mla_fwd_narrow(FwdParams p) {
    static_assert(HW * KW == kWaves, "narrow variant shape");
    using R = std::conditional_t<FP8, RingFp8<64>, Ring<64, 2>>;
    constexpr int kBN = R::BN;
    constexpr int RPW = kBN / KW;   // tile rows per wave
    constexpr int NSUB = RPW / 16;  // 16-row subtiles per wave
    static_assert(RPW == 16 || RPW == 32 || RPW == 64, "rows per wave");
    __shared__ __attribute__((aligned(1024))) char smem[R::LDS_BYTES];
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hw = wave % HW;
    const int kw = wave / HW;
    const int g = lane >> 4;
    const int n16 = lane & 15;

    const WgCoords c = wg_coords<kBN>(p);
    const int head = c.hgi * (16 * HW) + hw * 16 + n16;  // this lane's head
    // QK k-step ks (ks < 16) gives k-group g the 16-byte chunk 16 g + ks of the
    // 512 latent dims (Q and K agree; a dot product does not depend on the
    // order of its terms), so each k-group reads its own 256-byte window of
    // the row.  A ds_read_b128 serves the lanes 16 at a time, in quads: quad
    // q of a half-wave joins pass parity(popcount(q)) (measured on gfx950), so
    // a pass holds k-groups 0 and 1 (or 2 and 3) over complementary sets of 8
    // rows; with one window per k-group its 16 chunks are ks ^ sw_kv(row)
    // over all 16 rows -- 16 distinct bank groups.

    // Index loads first: the first gather depends on them, Q only on the
    // first MFMA.
    const IdxRegs<> ids = fetch_indices<kBN>(p, c);

    // ---- Q fragments: lane holds Q[head][128*g + 8*ks .. +7]; ks 16, 17 from
    // q_rope (dims 32*(ks-16) + 8*g).
    bf16x8 qf[18];
    {
        const uint16_t* qrow = p.q + ((int64_t)c.token * p.H + head) * 512 + 128 * g;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + 8 * ks);
        const uint16_t* rrow = p.q_rope + ((int64_t)c.token * p.H + head) * 64 + 8 * g;
        qf[16] = *reinterpret_cast<const bf16x8*>(rrow);
        qf[17] = *reinterpret_cast<const bf16x8*>(rrow + 32);
    }

    const uint32_t idx_lds = lds + R::IDX_OFF;
    store_indices<kBN>(ids, idx_lds, p, c);
    lds_barrier();
    const Gather gt = make_gather(p, c.b);
    const char* fp8_rows = fp8_base(p, c.b);
    auto issue = [&](int t) {
        if constexpr (FP8) issue_tile_fp8<R>(p, fp8_rows, t, R::raw(lds, t), idx_lds, wave, lane);
        else issue_tile<R>(p, gt, t, R::stage(lds, t), idx_lds, wave, lane);
    };

    // ---- per-lane LDS offsets (see the wide variant).
    const int rowbase = kw * RPW;
    // QK A operand: row rowbase + 16*s + n16, logical chunk 16*g + ks at byte
    // 256*g + ((ks ^ sw_kv(n16)) << 4) of the row.
    const uint32_t qk_g = (uint32_t)g << 8;
    const uint32_t qk_x = (uint32_t)sw_kv(n16) << 4;
    uint32_t rp_off[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) rp_off[j] = ((4 * j + g) ^ sw_rope(n16)) << 4;
    // PV A operand (transposed read): row rowbase + 32*k + 16*rd + 4*g + n16/4,
    // column 16*cb + 4*(n16 & 3) -> logical chunk 2*cb + ((n16 & 3) >> 1) =
    // 16*(cb>>3) + (2*(cb&7) + ((n16 & 3) >> 1)), byte 8*(n16 & 1) within it.
    const int tr_row = 4 * g + (n16 >> 2);
    uint32_t tr_off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) tr_off[j] = (((2 * j + ((n16 & 3) >> 1)) ^ sw_kv(tr_row)) << 4) + ((n16 & 1) << 3);

    // ---- running state (log2 units; see kRestartLog2)
    f32x4 oacc[32];
    float m_ref = -FLT_MAX;   // reference max of P
    float m_true = -FLT_MAX;  // exact running max
    float l_run = 0.f;        // per-lane partial of the head's sum, relative to m_ref
    const uint32_t flag_lds = lds + R::FLAG_OFF;

    // At most two passes over the range, as in the wide variant.
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int i = 0; i < 32; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    l_run = 0.f;
    if (pass == 1) m_ref = m_true;
    bool overflow = false;
    // One head slice (HW == 1) on bf16 rows: every wave gathers exactly the
    // rows it computes on (rows 16 w .. 16 w + 15 of each tile), so its
    // pipeline needs no workgroup barrier and keeps two tiles in flight,
    // issuing tile t + 2 into the stage it has just finished reading.
    constexpr bool kOwnRows = HW == 1 && !FP8;
    if (c.nt > 0) issue(0);
    wait_vmcnt<0>();  // Q and tile 0 (see the wide variant)
    if constexpr (kOwnRows)
        if (c.nt > 1) issue(1);

    for (int t = 0; t < c.nt; ++t) {
        if constexpr (kOwnRows) {
            if (t > 0) {  // tile t has landed; tile t + 1 may stay in flight
                if (t + 1 < c.nt) wait_vmcnt<R::LOADS_PER_TILE>();
                else wait_vmcnt<0>();
            }
        } else {
            wait_vmcnt<0>();  // this wave's gathers of tile t (two stages: nothing else in flight)
            lds_barrier();
            if (t + 1 < c.nt) issue(t + 1);
        }

        uint32_t stage, rope_rows;  // latent tile (bf16, swizzled); raw fp8 rows (rope)
        if constexpr (FP8) {
            if constexpr (HW == 1) {
                // one head slice: a wave alone reads its rows, so it expands
                // them itself and needs no barrier (LDS is in order per wave)
                dequant_rows(R::raw(lds, t), lds + R::KV_OFF, rowbase, lane);
            } else {
                dequant_tile<R>(R::raw(lds, t), lds + R::KV_OFF, wave, lane);
                lds_barrier();  // the expanded tile is complete
            }
            stage = lds + R::KV_OFF;
            rope_rows = R::raw(lds, t);
        } else {
            stage = R::stage(lds, t);
            rope_rows = 0;
        }
        // ---- S^T = K . Q^T for this wave's rows.  Steps run k-step major over
        // the NSUB subtiles in an explicit 4-deep LDS pipeline (the scheduler is
        // fenced per step); with one subtile the k-steps alternate between two
        // accumulators so consecutive MFMAs never depend on each other.
        // Slot indices of this lane's score rows, read before the MFMAs.
        i32x4 ivs[NSUB];
#pragma unroll
        for (int s = 0; s < NSUB; ++s) ivs[s] = lds_load<i32x4>(idx_lds + 4 * (t * kBN + rowbase + 16 * s + 4 * g));
        constexpr int QK_STEPS = 18 * NSUB;
        constexpr int NCH = NSUB == 1 ? 2 : 1;
        f32x4 sacc[NSUB][NCH];
#pragma unroll
        for (int s = 0; s < NSUB; ++s)
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) sacc[s][ch] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto kfrag = [&](int step) -> bf16x8 {
            const int ks = step / NSUB, s = step % NSUB;
            const int row = rowbase + 16 * s + n16;
            if (ks < 16) return lds_load<bf16x8>(stage + row * 1024 + qk_g + ((uint32_t)(16 * ks) ^ qk_x));
            if constexpr (FP8)
                return lds_load<bf16x8>(rope_rows + row * kFp8Row + kFp8RopeOff + ((4 * (ks - 16) + g) << 4));
            else
                return lds_load<bf16x8>(stage + R::KV_BYTES + row * 128 + rp_off[ks - 16]);
        };
        {
            bf16x8 kf[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) kf[j] = kfrag(j);
#pragma unroll
            for (int step = 0; step < QK_STEPS; ++step) {
                const int ks = step / NSUB, s = step % NSUB;
                const int ch = NCH == 2 ? (ks & 1) : 0;
                sacc[s][ch] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[step & 3], qf[ks], sacc[s][ch], 0, 0, 0);
                if (step + 4 < QK_STEPS) kf[step & 3] = kfrag(step + 4);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        f32x4 sres[NSUB];
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            sres[s] = sacc[s][0];
            if constexpr (NCH == 2) sres[s] += sacc[s][1];
        }

        // ---- scale, mask, online softmax.  Lane holds rows
        // rowbase + 16*s + 4*g + r (r = 0..3) of head n16.
        // Raw scores with masked rows at -inf; the scale folds into the max
        // and into one FMA per score (see the wide variant).
        float x[NSUB][4];
        float smax = -INFINITY;
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool valid = ivs[s][r] >= 0;
                x[s][r] = valid ? sres[s][r] : -INFINITY;
                smax = fmaxf(smax, x[s][r]);
            }
        }
        smax = max_xor32(max_xor16(smax));
        m_true = fmaxf(m_true, smax * p.score_scale_log2);
        if (m_ref == -FLT_MAX) m_ref = m_true;  // first valid rows: O and l are still zero
        const bool ovf = m_true > m_ref + kRestartLog2;
        overflow |= ovf;
        const float neg_ref = -m_ref;
        float psum = 0.f;
        bf16x4 pb[NSUB];
        if (__any(ovf)) {
            // This pass is to be discarded; the clamp keeps it free of inf.
#pragma unroll
            for (int s = 0; s < NSUB; ++s)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = fast_exp2(fminf(fmaf(x[s][r], p.score_scale_log2, neg_ref), kRestartLog2));
                    psum += e;
                    pb[s][r] = (__bf16)e;
                }
        } else {  // every P <= 2^kRestartLog2
#pragma unroll
            for (int s = 0; s < NSUB; ++s)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = fast_exp2(fmaf(x[s][r], p.score_scale_log2, neg_ref));
                    psum += e;
                    pb[s][r] = (__bf16)e;
                }
        }
        l_run += psum;

        // ---- O^T += V^T . P^T, one MFMA per (k-step, column block) in an
        // explicit LDS pipeline (PV_DEPTH fragments in flight).
        if constexpr (NSUB >= 2) {
            constexpr int PV_STEPS = (NSUB / 2) * 32;
            constexpr int PV_DEPTH = 4;
            bf16x8 pk[NSUB / 2];
#pragma unroll
            for (int k = 0; k < NSUB / 2; ++k)
                pk[k] = __builtin_shufflevector(pb[2 * k], pb[2 * k + 1], 0, 1, 2, 3, 4, 5, 6, 7);
            auto vfrag = [&](int step) -> bf16x8 {
                const int k = step >> 5, cb = step & 31;
                const uint32_t r0a = stage + (rowbase + 32 * k + tr_row) * 1024;
                const uint32_t pc = tr_off[cb & 7] + ((cb >> 3) << 8);
                const bf16x4 v0 = lds_load_tr(r0a + pc);
                const bf16x4 v1 = lds_load_tr(r0a + 16 * 1024 + pc);
                return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
            };
            bf16x8 vf[PV_DEPTH];
#pragma unroll
            for (int j = 0; j < PV_DEPTH; ++j) vf[j] = vfrag(j);
#pragma unroll
            for (int step = 0; step < PV_STEPS; ++step) {
                const int k = step >> 5, cb = step & 31;
                oacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[step % PV_DEPTH], pk[k], oacc[cb], 0, 0, 0);
                if (step + PV_DEPTH < PV_STEPS) vf[step % PV_DEPTH] = vfrag(step + PV_DEPTH);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            constexpr int PV_DEPTH = 8;
            const i16x4 pk = __builtin_bit_cast(i16x4, pb[0]);
            const uint32_t r0a = stage + (rowbase + tr_row) * 1024;
            auto vfrag = [&](int cb) -> i16x4 {
                return __builtin_bit_cast(i16x4, lds_load_tr(r0a + tr_off[cb & 7] + ((cb >> 3) << 8)));
            };
            i16x4 vf[PV_DEPTH];
#pragma unroll
            for (int j = 0; j < PV_DEPTH; ++j) vf[j] = vfrag(j);
#pragma unroll
            for (int cb = 0; cb < 32; ++cb) {
                oacc[cb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf[cb % PV_DEPTH], pk, oacc[cb], 0, 0, 0);
                if (cb + PV_DEPTH < 32) vf[cb % PV_DEPTH] = vfrag(cb + PV_DEPTH);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (kOwnRows)
            if (t + 2 < c.nt) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's reads of the stage are done
                issue(t + 2);
            }
    }

    // ---- workgroup vote: does any head need pass 1?
    if (pass == 1) break;
    if (threadIdx.x == 0) lds_store<int>(flag_lds, 0);
    lds_barrier();  // also: every wave is past its last ring read
    if (__any(overflow) && lane == 0) lds_store<int>(flag_lds, 1);
    lds_barrier();
    if (__builtin_amdgcn_readfirstlane(lds_load<int>(flag_lds)) == 0) break;
    }

    // ---- epilogue
    l_run = sum_xor32(sum_xor16(l_run));
    int cb_lo = 0, cb_hi = 32;

    if constexpr (KW > 1) {
        // Merge the KW row-split waves of each head slice through LDS (same
        // FP32 merge as the split merge): M = max m_ref_k, w_k = exp(m_ref_k - M).
        constexpr int OX_STRIDE = 516;  // floats per head row (padded)
        static_assert(kWaves * 16 * OX_STRIDE * 4 <= R::IDX_OFF, "exchange fits the ring");
        lds_barrier();  // every wave is past its last ring read
        const uint32_t ml = lds + R::IDX_OFF;  // [3][4 waves][16] floats: m_ref, m_true, l
        if (g == 0) {
            lds_store<float>(ml + 4 * (wave * 16 + n16), m_ref);
            lds_store<float>(ml + 4 * (kWaves * 16 + wave * 16 + n16), m_true);
            lds_store<float>(ml + 4 * (2 * kWaves * 16 + wave * 16 + n16), l_run);
        }
        // Head row (wave, n16): column group g of block cb at float 128 g + 4 cb,
        // so a lane's bank group is set by its row alone (rows are 129 chunks
        // apart) and each 16-lane pass of ds_write/read_b128 -- k-groups 0 and 1
        // over complementary rows -- touches 16 distinct bank groups.
        const uint32_t ox = lds + ((wave * 16 + n16) * OX_STRIDE + 128 * g) * 4;
#pragma unroll
        for (int cb = 0; cb < 32; ++cb) lds_store<f32x4>(ox + cb * 16, oacc[cb]);
        lds_barrier();
        float mk[KW], lk[KW];
        float mref = -FLT_MAX, mtrue = -FLT_MAX;
#pragma unroll
        for (int k = 0; k < KW; ++k) {
            const int wk = k * HW + hw;
            mk[k] = lds_load<float>(ml + 4 * (wk * 16 + n16));
            mtrue = fmaxf(mtrue, lds_load<float>(ml + 4 * (kWaves * 16 + wk * 16 + n16)));
            lk[k] = lds_load<float>(ml + 4 * (2 * kWaves * 16 + wk * 16 + n16));
            mref = fmaxf(mref, mk[k]);
        }
        float lsum = 0.f;
        float wgt[KW];
#pragma unroll
        for (int k = 0; k < KW; ++k) {
            wgt[k] = fast_exp2(mk[k] - mref);
            lsum += wgt[k] * lk[k];
        }
        m_ref = mref;
        m_true = mtrue;
        l_run = lsum;
        // wave kw finishes columns [cb_lo, cb_hi) of its head slice
        cb_lo = kw * (32 / KW);
        cb_hi = cb_lo + 32 / KW;
#pragma unroll
        for (int cb = 0; cb < 32; ++cb) {
            if (cb >= cb_lo && cb < cb_hi) {  // uniform branch; keeps oacc in registers
                f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < KW; ++k) {
                    const int wk = k * HW + hw;
                    const f32x4 v = lds_load<f32x4>(lds + ((wk * 16 + n16) * OX_STRIDE + 128 * g + 4 * cb) * 4);
                    acc += wgt[k] * v;
                }
                oacc[cb] = acc;
            }
        }
    }

    // Re-express (m_ref, l, O) against the true max for the caller.
    const float to_true = fast_exp2(m_ref - m_true);
    const float l_fin = l_run * to_true;
    const float m_nat = m_true * kLn2;
    if (p.nsplit == 1) {
        const float inv_l = 1.0f / l_run;  // O and l_run share m_ref
        uint16_t* orow = p.out + ((int64_t)c.token * p.H + head) * 512 + 4 * g;
#pragma unroll
        for (int cb = 0; cb < 32; ++cb)
            if (cb >= cb_lo && cb < cb_hi)
                store_bf16x4(orow + 16 * cb, oacc[cb][0] * inv_l, oacc[cb][1] * inv_l, oacc[cb][2] * inv_l,
                             oacc[cb][3] * inv_l);
        if (g == 0 && kw == 0) {
            p.out_max[(int64_t)c.token * p.H + head] = m_nat;
            p.out_sum[(int64_t)c.token * p.H + head] = l_fin;
        }
    } else if (p.arrivals == nullptr) {
        const int64_t prow = ((int64_t)c.token * p.nsplit + c.sp) * p.H + head;
        float* orow = p.part_o + prow * 512 + 4 * g;
#pragma unroll
        for (int cb = 0; cb < 32; ++cb)
            if (cb >= cb_lo && cb < cb_hi) *reinterpret_cast<f32x4*>(orow + 16 * cb) = oacc[cb] * to_true;
        if (g == 0 && kw == 0) {
            p.part_m[prow] = m_nat;
            p.part_l[prow] = l_fin;
        }
    } else {
        // In-kernel merge: the same partials, stored agent-coherent.
        constexpr int kHeads = 16 * HW;
        const int head0 = c.hgi * kHeads, hl = hw * 16 + n16;
        const __amdgpu_buffer_rsrc_t rs = group_block(p, c.token, c.sp, head0, kHeads);
        const uint32_t voff = (uint32_t)(hl * 2048 + 16 * g);
#pragma unroll
        for (int cb = 0; cb < 32; ++cb)
            if (cb >= cb_lo && cb < cb_hi)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, oacc[cb] * to_true), rs,
                                                       voff + 64 * cb, 0, kAgentCoherent);
        if (g == 0 && kw == 0) {
            const int64_t prow = ((int64_t)c.token * p.nsplit + c.sp) * p.H + head;
            __hip_atomic_store(p.part_m + prow, m_nat, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.part_l + prow, l_fin, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        merge_if_last<32 / KW>(p, c, head0, kHeads, hl, g, g == 0 && kw == 0, cb_lo, flag_lds);
    }
}

// ============================================================ column-split PV
// pv_cols = 128.  The four waves split each 64-row tile's ROWS for QK and the
// softmax (wave w: rows 16 w .. 16 w + 15), exchange the bf16 P tile through
// LDS, and split the 512 output COLUMNS for PV (wave w: columns 128 w ..
// 128 w + 127, over all 64 rows of the tile).  A wave holds HB head blocks of
// 16 (v_mfma_f32_16x16x32_bf16; each K and V fragment read from LDS serves all
// HB blocks), so every gathered element is read from LDS once for QK and once
// for PV whatever the head count; PV runs with k = 32 rows (full MFMA rate); and
// no O accumulators are exchanged at the end, each wave owning its own output
// columns.  The four waves share one reference max per head, fixed from the
// first tile with a valid row (the restart logic of the other variants applies
// unchanged to it).
//
// PROD adds four gather waves (waves 4..7, one per SIMD beside a compute
// wave): a wave stalls while the texture path accepts its row loads (≈0.7 us
// per 64-row tile at ≈50 B/clk per CU), and with separate gather waves that
// stall no longer holds up the compute waves' MFMAs.  The gather waves pass
// every workgroup barrier the compute waves pass (they mirror the
// reference-max exchange from the same LDS values) and hold no accumulators.
// The 16-head kernel fits 2 waves per SIMD (252 VGPRs, no spills); the 32-
// and 64-head kernels do not and run without gather waves.
template <int HB>
struct XpLds {
    static constexpr int BM = 16 * HB;
    static constexpr int RING = 2 * 64 * 1152;
    static constexpr int IDX_CAP = HB <= 2 ? DSA_IDX_CAP : DSA_IDX_CAP / 2;
    static constexpr int IDX_OFF = RING;
    // P of one tile, per head 64 bf16 in the k order of the PV B operand
    // (position 32 kk + 8 g + 4 a + j holds row 32 kk + 16 a + 4 g + j), heads
    // 144 bytes apart.
    static constexpr int P_STRIDE = 144;
    static constexpr int P_OFF = IDX_OFF + IDX_CAP * 4;
    static constexpr int MX_OFF = P_OFF + BM * P_STRIDE;  // [4 waves][BM] floats
    static constexpr int FLAG_OFF = MX_OFF + kWaves * BM * 4;
    static constexpr int LDS_BYTES = FLAG_OFF + 16;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(2 * kWaves * BM * 4 <= RING, "epilogue exchange fits the ring");
};

template <int HB, bool PROD>
__global__ __launch_bounds__(PROD ? 2 * kThreads : kThreads, 1) void sparse_mla_fwd_xp(FwdParams p) {
    using R = Ring<64, 2>;
    using X = XpLds<HB>;
    constexpr int kBN = 64;
    __shared__ __attribute__((aligned(1024))) char smem[X::LDS_BYTES];
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // With PROD, waves 4..7 only gather (wave 4 + w fetches what wave w
    // would) and keep the workgroup barriers in step with the compute waves.
    const bool producer = PROD && wave >= kWaves;
    const int gw = producer ? wave - kWaves : wave;
    const int g = lane >> 4;
    const int n16 = lane & 15;

    const WgCoords c = wg_coords<kBN>(p);
    const int head0 = c.hgi * X::BM;
    IdxRegs<X::IDX_CAP> ids;
    if (!producer) ids = fetch_indices<kBN, X::IDX_CAP>(p, c);

    // ---- Q fragments of the HB head blocks (as in the narrow variant):
    // lane holds Q[head][128 g + 8 ks .. + 7]; ks 16, 17 from q_rope.
    bf16x8 qf[HB][18];
#pragma unroll
    for (int hb = 0; hb < (producer ? 0 : HB); ++hb) {
        const int head = head0 + hb * 16 + n16;
        const uint16_t* qrow = p.q + ((int64_t)c.token * p.H + head) * 512 + 128 * g;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qf[hb][ks] = *reinterpret_cast<const bf16x8*>(qrow + 8 * ks);
        const uint16_t* rrow = p.q_rope + ((int64_t)c.token * p.H + head) * 64 + 8 * g;
        qf[hb][16] = *reinterpret_cast<const bf16x8*>(rrow);
        qf[hb][17] = *reinterpret_cast<const bf16x8*>(rrow + 32);
    }

    const uint32_t idx_lds = lds + X::IDX_OFF;
    if (!producer) store_indices<kBN>(ids, idx_lds, p, c);
    lds_barrier();
    const Gather gt = make_gather(p, c.b);

    // QK A operand: row 16 wave + n16, logical chunk 16 g + ks (sw_kv depends
    // on the row mod 16 only).
    const uint32_t qk_g = (uint32_t)g << 8;
    const uint32_t qk_x = (uint32_t)sw_kv(n16) << 4;
    uint32_t rp_off[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) rp_off[j] = ((4 * j + g) ^ sw_rope(n16)) << 4;
    // PV A operand (transposed reads, as in the narrow variant) restricted to
    // this wave's 256-byte column window.
    const int tr_row = 4 * g + (n16 >> 2);
    uint32_t tr_off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        tr_off[j] = ((((2 * j + ((n16 & 3) >> 1)) ^ sw_kv(tr_row)) << 4) + ((n16 & 1) << 3)) + ((uint32_t)wave << 8);
    // P exchange: this wave writes rows 16 wave + 4 g .. + 3 of head n16 (8
    // bytes) and reads positions 32 kk + 8 g .. + 7 (16 bytes) for the PV B
    // operand.
    const uint32_t p_base = lds + X::P_OFF + (uint32_t)n16 * X::P_STRIDE;
    const uint32_t p_wr = p_base + (uint32_t)(32 * (wave >> 1) + 8 * g + 4 * (wave & 1)) * 2;
    const uint32_t p_rd = p_base + (uint32_t)(8 * g) * 2;
    const uint32_t mx_lds = lds + X::MX_OFF;
    const uint32_t flag_lds = lds + X::FLAG_OFF;

    // ---- running state, per head block (log2 units)
    f32x4 oacc[HB][8];
    float m_ref[HB], m_true[HB], l_run[HB];
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) m_ref[hb] = m_true[hb] = -FLT_MAX;

#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) oacc[hb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
            l_run[hb] = 0.f;
        }
        bool ref_set = pass == 1;  // pass 1 runs against the exact max (set at the vote)
        bool overflow = false;
        if (!PROD || producer) issue_tile<R>(p, gt, 0, R::stage(lds, 0), idx_lds, gw, lane);
        wait_vmcnt<0>();  // Q and tile 0

        for (int t = 0; t < c.nt; ++t) {
            if (t > 0) wait_vmcnt<0>();  // this wave's gathers of tile t
            lds_barrier();                // tile t complete; stage of tile t - 1, P and MX free
            if (t + 1 < c.nt && (!PROD || producer))
                issue_tile<R>(p, gt, t + 1, R::stage(lds, t + 1), idx_lds, gw, lane);
            if (producer) {
                // The compute waves' barriers of this tile: the reference max
                // exchange (same decision, from the same LDS values) and P.
                if (!ref_set) {
                    lds_barrier();
                    float t0 = -INFINITY;
#pragma unroll
                    for (int w = 0; w < kWaves; ++w) t0 = fmaxf(t0, lds_load<float>(mx_lds + 4 * (w * X::BM)));
                    if (__builtin_amdgcn_readfirstlane(__float_as_int(t0)) != __float_as_int(-INFINITY)) ref_set = true;
                }
                lds_barrier();
                continue;
            }
            const uint32_t stage = R::stage(lds, t);

            // ---- S^T = K . Q^T for this wave's 16 rows and HB head blocks.
            const i32x4 iv = lds_load<i32x4>(idx_lds + 4 * (t * kBN + 16 * wave + 4 * g));
            const uint32_t krow = stage + (uint32_t)(16 * wave + n16) * 1024;
            auto kfrag = [&](int ks) -> bf16x8 {
                if (ks < 16) return lds_load<bf16x8>(krow + qk_g + ((uint32_t)(16 * ks) ^ qk_x));
                return lds_load<bf16x8>(stage + R::KV_BYTES + (16 * wave + n16) * 128 + rp_off[ks - 16]);
            };
            constexpr int NCH = HB == 1 ? 2 : 1;
            f32x4 sacc[HB][NCH];
#pragma unroll
            for (int hb = 0; hb < HB; ++hb)
#pragma unroll
                for (int ch = 0; ch < NCH; ++ch) sacc[hb][ch] = f32x4{0.f, 0.f, 0.f, 0.f};
            {
                bf16x8 kf[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) kf[j] = kfrag(j);
#pragma unroll
                for (int ks = 0; ks < 18; ++ks) {
                    const int ch = NCH == 2 ? (ks & 1) : 0;
#pragma unroll
                    for (int hb = 0; hb < HB; ++hb)
                        sacc[hb][ch] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks & 3], qf[hb][ks], sacc[hb][ch], 0, 0, 0);
                    if (ks + 4 < 18) kf[ks & 3] = kfrag(ks + 4);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }

            // ---- scale, mask, max over this wave's rows; lane holds rows
            // 16 wave + 4 g + r (r = 0..3) of head hb * 16 + n16.
            float x[HB][4], lmax[HB];
#pragma unroll
            for (int hb = 0; hb < HB; ++hb) {
                f32x4 sres = sacc[hb][0];
                if constexpr (NCH == 2) sres += sacc[hb][1];
                lmax[hb] = -INFINITY;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    x[hb][r] = iv[r] >= 0 ? sres[r] : -INFINITY;
                    lmax[hb] = fmaxf(lmax[hb], x[hb][r]);
                }
                lmax[hb] = max_xor32(max_xor16(lmax[hb])) * p.score_scale_log2;
                m_true[hb] = fmaxf(m_true[hb], lmax[hb]);
            }
            if (!ref_set) {
                // The first tile with a valid row fixes the shared reference
                // max: the tile's max per head over all four waves.
                if (g == 0)
#pragma unroll
                    for (int hb = 0; hb < HB; ++hb) lds_store<float>(mx_lds + 4 * (wave * X::BM + hb * 16 + n16), lmax[hb]);
                lds_barrier();
                float tmax[HB];
#pragma unroll
                for (int hb = 0; hb < HB; ++hb) {
                    tmax[hb] = -INFINITY;
#pragma unroll
                    for (int w = 0; w < kWaves; ++w)
                        tmax[hb] = fmaxf(tmax[hb], lds_load<float>(mx_lds + 4 * (w * X::BM + hb * 16 + n16)));
                }
                // a tile either has a valid row (every head's max is finite) or not
                if (__builtin_amdgcn_readfirstlane(__float_as_int(tmax[0])) != __float_as_int(-INFINITY)) {
#pragma unroll
                    for (int hb = 0; hb < HB; ++hb) m_ref[hb] = tmax[hb];
                    ref_set = true;
                }
            }
            bool ovf = false;
#pragma unroll
            for (int hb = 0; hb < HB; ++hb) ovf |= lmax[hb] > m_ref[hb] + kRestartLog2;
            overflow |= ovf;
            bf16x4 pb[HB];
            const bool clamp = __any(ovf);
#pragma unroll
            for (int hb = 0; hb < HB; ++hb) {
                const float neg_ref = -m_ref[hb];
                float psum = 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a = fmaf(x[hb][r], p.score_scale_log2, neg_ref);
                    const float e = fast_exp2(clamp ? fminf(a, kRestartLog2) : a);
                    psum += e;
                    pb[hb][r] = (__bf16)e;
                }
                l_run[hb] += psum;
                lds_store<bf16x4>(p_wr + hb * 16 * X::P_STRIDE, pb[hb]);
            }
            lds_barrier();  // P of all four waves

            // ---- O^T[cols of this wave] += V^T . P^T over the tile's 64 rows:
            // 2 k-steps x 8 column blocks, each V fragment used by HB MFMAs.
            bf16x8 pk[HB][2];
#pragma unroll
            for (int hb = 0; hb < HB; ++hb)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    pk[hb][kk] = lds_load<bf16x8>(p_rd + hb * 16 * X::P_STRIDE + kk * 64);
            auto vfrag = [&](int step) -> bf16x8 {
                const int kk = step >> 3, cb = step & 7;
                const uint32_t r0a = stage + (uint32_t)(32 * kk + tr_row) * 1024 + tr_off[cb];
                const bf16x4 v0 = lds_load_tr(r0a);
                const bf16x4 v1 = lds_load_tr(r0a + 16 * 1024);
                return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
            };
            constexpr int PV_DEPTH = 4;
            bf16x8 vf[PV_DEPTH];
#pragma unroll
            for (int j = 0; j < PV_DEPTH; ++j) vf[j] = vfrag(j);
#pragma unroll
            for (int step = 0; step < 16; ++step) {
                const int kk = step >> 3, cb = step & 7;
#pragma unroll
                for (int hb = 0; hb < HB; ++hb)
                    oacc[hb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[step % PV_DEPTH], pk[hb][kk], oacc[hb][cb], 0, 0, 0);
                if (step + PV_DEPTH < 16) vf[step % PV_DEPTH] = vfrag(step + PV_DEPTH);
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        // ---- workgroup vote: does any head need pass 1?
        if (pass == 1) break;
        if (threadIdx.x == 0) lds_store<int>(flag_lds, 0);
        lds_barrier();  // also: every wave is past its last ring and P read
        if (__any(overflow) && lane == 0) lds_store<int>(flag_lds, 1);
        lds_barrier();
        if (__builtin_amdgcn_readfirstlane(lds_load<int>(flag_lds)) == 0) break;
        // pass 1 runs against the exact max over all waves
        if (g == 0 && !producer)
#pragma unroll
            for (int hb = 0; hb < HB; ++hb) lds_store<float>(mx_lds + 4 * (wave * X::BM + hb * 16 + n16), m_true[hb]);
        lds_barrier();
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            float mt = -FLT_MAX;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) mt = fmaxf(mt, lds_load<float>(mx_lds + 4 * (w * X::BM + hb * 16 + n16)));
            m_ref[hb] = mt;
        }
        lds_barrier();  // MX read by every wave before any tile writes it again
    }

    // ---- epilogue: sum l and take the max over the four waves' rows (the ring
    // is free once every wave is past its last read).
    lds_barrier();
    constexpr int kPartOff = 4096;  // staged partial rows, past the l / max exchange
    static_assert(kPartOff + X::BM * kPartRow <= X::RING, "staged partials fit the ring");
    if (producer) {
        // the compute waves' remaining barriers; the partial rows' stores
        // are shared by all eight waves
        lds_barrier();
        if (p.nsplit == 1) {
            lds_barrier();
        } else {
            lds_barrier();  // rows staged
            if (HB > 1 || p.arrivals == nullptr) {
                store_staged_partials<kPartPlain>(p, c, head0, X::BM, lds + kPartOff, wave, 2 * kWaves, lane);
            } else {
                store_staged_partials<kPartAgent>(p, c, head0, X::BM, lds + kPartOff, wave, 2 * kWaves, lane);
                wait_vmcnt<0>();  // the count-in's barriers (group_count_in)
                lds_barrier();
                lds_barrier();
            }
        }
        return;
    }
    const uint32_t l_lds = lds, mt_lds = lds + kWaves * X::BM * 4;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
        l_run[hb] = sum_xor32(sum_xor16(l_run[hb]));
        if (g == 0) {
            lds_store<float>(l_lds + 4 * (wave * X::BM + hb * 16 + n16), l_run[hb]);
            lds_store<float>(mt_lds + 4 * (wave * X::BM + hb * 16 + n16), m_true[hb]);
        }
    }
    lds_barrier();
    int eln = lane;
    asm volatile("" : "+v"(eln));
    const int eg = eln >> 4, en16 = eln & 15;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
        float lt = 0.f, mt = -FLT_MAX;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            lt += lds_load<float>(l_lds + 4 * (w * X::BM + hb * 16 + en16));
            mt = fmaxf(mt, lds_load<float>(mt_lds + 4 * (w * X::BM + hb * 16 + en16)));
        }
        l_run[hb] = lt;
        m_true[hb] = mt;
    }
    const bool writes_ml = wave == 0 && eg == 0;
    if (p.nsplit == 1) {
        // bf16 rows staged in the ring past the l / max exchange, then stored
        // one whole 1 KiB head row per instruction (a lane holds 4 columns of
        // 8 column blocks: 8-byte pieces 32 bytes apart in memory).
        constexpr int HROW = 1040;  // bytes per staged head row (1 KiB + 16: spreads heads over the banks)
        constexpr int STAGE_OFF = 4096;
        static_assert(2 * kWaves * X::BM * 4 <= STAGE_OFF && STAGE_OFF + X::BM * HROW <= X::RING, "staging fits");
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            const int head = head0 + hb * 16 + en16;
            const float inv_l = 1.0f / l_run[hb];  // O and l share m_ref
            const uint32_t srow = lds + STAGE_OFF + (uint32_t)((hb * 16 + en16) * HROW + 2 * (128 * wave + 4 * eg));
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) {
                bf16x4 v;
                v[0] = (__bf16)(oacc[hb][cb][0] * inv_l);
                v[1] = (__bf16)(oacc[hb][cb][1] * inv_l);
                v[2] = (__bf16)(oacc[hb][cb][2] * inv_l);
                v[3] = (__bf16)(oacc[hb][cb][3] * inv_l);
                lds_store<bf16x4>(srow + 2 * 16 * cb, v);
            }
            if (writes_ml) {
                p.out_max[(int64_t)c.token * p.H + head] = m_true[hb] * kLn2;
                p.out_sum[(int64_t)c.token * p.H + head] = l_run[hb] * fast_exp2(m_ref[hb] - m_true[hb]);
            }
        }
        lds_barrier();
        // wave w stores head rows w, w + 4, ...: 64 lanes x 16 bytes = one row
        uint16_t* obase = p.out + ((int64_t)c.token * p.H + head0) * 512 + 8 * eln;
#pragma unroll
        for (int hr = wave; hr < X::BM; hr += kWaves)
            *reinterpret_cast<bf16x8*>(obase + (int64_t)hr * 512) =
                lds_load<bf16x8>(lds + STAGE_OFF + hr * HROW + 16 * eln);
    } else {
        // FP32 partial rows staged past the l / max exchange, then stored as
        // whole 1 KiB halves by every wave; with the in-kernel merge they and
        // m / l are stored agent-coherent and the last workgroup of the
        // (token, head group) merges.
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            const int head = head0 + hb * 16 + en16;
            const float to_true = fast_exp2(m_ref[hb] - m_true[hb]);
            const uint32_t srow = lds + kPartOff + (uint32_t)((hb * 16 + en16) * kPartRow + 4 * (128 * wave + 4 * eg));
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) lds_store<f32x4>(srow + 64 * cb, oacc[hb][cb] * to_true);
            if (writes_ml) {
                const int64_t prow = ((int64_t)c.token * p.nsplit + c.sp) * p.H + head;
                if (HB > 1 || p.arrivals == nullptr) {
                    p.part_m[prow] = m_true[hb] * kLn2;
                    p.part_l[prow] = l_run[hb] * to_true;
                } else {
                    __hip_atomic_store(p.part_m + prow, m_true[hb] * kLn2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(p.part_l + prow, l_run[hb] * to_true, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        lds_barrier();  // rows staged
        constexpr int kStoreWaves = PROD ? 2 * kWaves : kWaves;
        if (HB > 1 || p.arrivals == nullptr) {
            store_staged_partials<kPartPlain>(p, c, head0, X::BM, lds + kPartOff, wave, kStoreWaves, eln);
        } else {
            store_staged_partials<kPartAgent>(p, c, head0, X::BM, lds + kPartOff, wave, kStoreWaves, eln);
            merge_if_last<8>(p, c, head0, 16, en16, eg, writes_ml, 8 * wave, flag_lds);
        }
    }
}

// Byte offset of k-group g's 16-byte P chunk of head h (within a 64-head
// buffer).  With 64-byte heads, the lanes of one ds_read_b128 / ds_write_b128
// pass (four quads of a half-wave, chosen by popcount parity) would meet 4
// heads apart on the same banks; XOR-ing the chunk with f(h / 4) =
// {0, 2, 3, 1} gives every pass 16 distinct bank groups.
__device__ __forceinline__ uint32_t pp_pchunk(int h, int g) {
    return (uint32_t)(h * 64 + 16 * (g ^ ((0x78 >> (2 * ((h >> 2) & 3))) & 3)));
}

// ====================================================== specialised waves
// 16 or 32 heads per workgroup (HB head blocks of 16), 32-row tiles in a
// 4-stage ring, and waves with fixed roles (wave w runs on SIMD w % 4):
//   waves 0 .. HB-1      QK + softmax: wave hb scores the tile's 32 rows
//                        against head block hb (Q in registers) and writes
//                        its bf16 P into P buffer s % 2;
//   waves HB, HB+1       PV: wave v accumulates O for columns 256 v ..
//                        256 v + 255 of all HB head blocks over tile s - 1
//                        (one 16x16x32 MFMA per 16-column block and head
//                        block);
//   waves HB+2 .. HB+5   gathers: gather wave j loads kv rows 8 j .. 8 j + 7
//                        of a tile and their rope rows into registers
//                        (ordinary buffer loads, three tiles ahead) and writes
//                        tile s + 2 into its ring stage during step s.
// Steps s = 0 .. nt are separated by one workgroup barrier each.  A wave
// stalls while the texture path accepts its loads; here only the gather
// waves stall, and with three tiles of rows in their registers the load
// latency hides behind the steps in between.  Tile t occupies stage t % 4
// from step t - 2 (written) to step t + 1 (its PV); P(t) is written in step t
// and read in step t + 1.  A QK wave owns every row of its 16 heads, so its
// reference max is its own (set at its first valid rows, as in the ping-pong
// kernel) and the restart logic applies unchanged.  Split merge: the merge
// kernel, or for 16 heads (arrival counters given) in the workgroup of each
// (token, head group) that stores its partials last, as the column-split
// kernel does (merge_if_last).
// Fragment pipelines: 10 K reads (QK) and 6 V fragment pairs (PV) in flight
// per wave (with the k-order of qk_lane_chunk, 10 beat 8, 12 and 14 by
// 0.4 % at C2; PV 4 and 8 measured the same as 6).
#ifndef XS_QK_DEPTH
#define XS_QK_DEPTH 10
#endif
#ifndef XS_PV_DEPTH
#define XS_PV_DEPTH 6
#endif
template <int HB>
struct XsLds {
    static constexpr int BN = 32, NSTAGE = 4;
    static constexpr int KV_BYTES = BN * 1024;
    static constexpr int STAGE_BYTES = BN * 1152;
    static constexpr int IDX_OFF = NSTAGE * STAGE_BYTES;
    // P of one tile: 16 HB heads x 32 bf16 in the k order of the PV B operand
    // (position 8 g + j holds tile row 4 g + j for j < 4, 16 + 4 g + j - 4
    // otherwise), 64 bytes per head; the 16-byte chunk of k-group g of head h
    // sits at pp_pchunk(h, g).
    static constexpr int P_OFF = IDX_OFF + DSA_IDX_CAP * 4;
    static constexpr int P_BYTES = 16 * HB * 64;
    static constexpr int EPI_OFF = P_OFF + 2 * P_BYTES;  // l, reference max, max: [3][16 HB] floats
    static constexpr int FLAG_OFF = EPI_OFF + 3 * 16 * HB * 4;
    static constexpr int LDS_BYTES = FLAG_OFF + 16;
    static constexpr int WAVES = HB + 6;
    static constexpr int DEPTH = 3;  // tiles held in the gather waves' registers
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    __device__ static uint32_t stage(uint32_t lds, int t) { return lds + (uint32_t)(t % NSTAGE) * STAGE_BYTES; }
};

// One gather wave's share of a tile in registers: kv rows 8 j .. 8 j + 7
// (lane l holds bytes (16 l) ^ (16 sw_kv(row)) of each) and one 16-byte chunk
// of rope rows 8 j + l / 8.
struct XsRows {
    u32x4 v[9];
};

// Loads of tile t.  Tiles past the range load nothing (an empty descriptor:
// the loads still issue, so the compiler's wait counts stay exact) and read
// the index cache of the last tile.
__device__ __forceinline__ void xs_load(const FwdParams& p, const char* kv, const char* kr, int t, int nt,
                                        uint32_t idx_lds, int j, int lane, XsRows& b) {
    const bool live = t < nt;
    const int tt = max(min(t, nt - 1), 0);
    const int rows = p.kv_rows;
    const int r0 = 8 * j;
    const int my_id = lds_load<int>(idx_lds + 4 * (tt * XsLds<1>::BN + r0 + (lane & 7)));
    const uint32_t my_row = (uint32_t)min(max(my_id, 0), rows - 1);
    const uint32_t lane16 = (uint32_t)lane << 4;
    const int row_bytes = live ? 1024 : 0;
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
        const uint32_t row = __builtin_amdgcn_readlane(my_row, rr);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char*>(kv) + ((uint64_t)row << 10), (short)0, row_bytes, 0x00020000);
        b.v[rr] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane16 ^ ((uint32_t)sw_kv(r0 + rr) << 4), 0, 0);
    }
    const int r = r0 + (lane >> 3);
    const int id = lds_load<int>(idx_lds + 4 * (tt * XsLds<1>::BN + r));
    const uint32_t voff = ((uint32_t)min(max(id, 0), rows - 1) << 7) + (((lane & 7) ^ sw_rope(r)) << 4);
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(kr), (short)0, live ? (int)((uint32_t)rows * 128u) : 0, 0x00020000);  // < 2^32 bytes
    b.v[8] = __builtin_amdgcn_raw_buffer_load_b128(rr, voff, 0, 0);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order: the loads of later tiles stay in flight
}
// The same rows into the stage of tile t (the layout the LDS-DMA gathers of
// the other variants produce).
__device__ __forceinline__ void xs_store(uint32_t stage, int j, int lane, const XsRows& b) {
    const uint32_t st = stage + ((uint32_t)lane << 4);
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) lds_store<u32x4>(st + (8 * j + rr) * 1024, b.v[rr]);
    lds_store<u32x4>(st + XsLds<1>::KV_BYTES + 8 * j * 128, b.v[8]);  // ring layout: the same for every HB
    __builtin_amdgcn_sched_barrier(0);
}

template <int HB>
__global__ __launch_bounds__(64 * XsLds<HB>::WAVES, 1) void sparse_mla_fwd_xs(FwdParams p) {
    using X = XsLds<HB>;
    constexpr int BN = X::BN;
    constexpr int BM = 16 * HB;
    __shared__ __attribute__((aligned(1024))) char smem[X::LDS_BYTES];
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;
    const int n16 = lane & 15;

    const WgCoords c = wg_coords<BN>(p);
    const int head0 = c.hgi * BM;
    const uint32_t idx_lds = lds + X::IDX_OFF;
    const uint32_t p_lds = lds + X::P_OFF;
    const uint32_t epi = lds + X::EPI_OFF;
    const uint32_t flag_lds = lds + X::FLAG_OFF;

    // Index loads (threads 0..255: QK, PV and the first gather waves).
    // Indices masked and in LDS before the Q loads issue: deferring them
    // behind Q (as the other kernels do) measured 0.35 us slower at C2.
    if (wave < 4) store_indices<BN>(fetch_indices<BN>(p, c), idx_lds, p, c);
    // Q of the QK wave's head block: lane holds Q[head][32 ks + 8 qk_lane_chunk(g)
    // .. + 7]; ks 16, 17 from q_rope (dims 32 (ks - 16) + 8 g).
    bf16x8 qf[18];
    if (wave < HB) {
        const int head = head0 + 16 * wave + n16;
        const uint16_t* qrow = p.q + ((int64_t)c.token * p.H + head) * 512 + 8 * qk_lane_chunk(g);
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + 32 * ks);
        const uint16_t* rrow = p.q_rope + ((int64_t)c.token * p.H + head) * 64 + 8 * g;
        qf[16] = *reinterpret_cast<const bf16x8*>(rrow);
        qf[17] = *reinterpret_cast<const bf16x8*>(rrow + 32);
    }
    lds_barrier();

    // Second-pass vote (every wave): the flag is raised by a QK wave whose
    // scores outgrew its reference max by more than kRestartLog2.
    auto vote = [&](bool overflow) -> bool {
        if (threadIdx.x == 0) lds_store<int>(flag_lds, 0);
        lds_barrier();
        if (__any(overflow) && lane == 0) lds_store<int>(flag_lds, 1);
        lds_barrier();
        return __builtin_amdgcn_readfirstlane(lds_load<int>(flag_lds)) != 0;
    };
    // End of every wave, after the PV waves' epilogue.  Split 1: the output
    // rows staged by the PV waves; wave w stores head rows w, w + WAVES, ...:
    // 64 lanes x 16 bytes = one row.  In-kernel merge (16 heads): every wave
    // counts in; true in the group's last workgroup, where the PV waves then
    // merge their columns.
    auto finish = [&]() -> bool {
        if (p.nsplit == 1) {
            lds_barrier();  // rows staged
            uint16_t* obase = p.out + ((int64_t)c.token * p.H + head0) * 512 + 8 * lane;
            for (int hr = wave; hr < BM; hr += X::WAVES)
                *reinterpret_cast<bf16x8*>(obase + (int64_t)hr * 512) =
                    lds_load<bf16x8>(lds + hr * 1040 + 16 * lane);
            return false;
        }
        // FP32 partial rows staged in the ring, stored as whole 1 KiB halves
        static_assert(BM * kPartRow <= X::IDX_OFF, "staged partials fit the ring");
        lds_barrier();  // rows staged
        if (HB > 1 || p.arrivals == nullptr) {
            store_staged_partials<kPartNonTemporal>(p, c, head0, BM, lds, wave, X::WAVES, lane);
            return false;
        }
        store_staged_partials<kPartAgent>(p, c, head0, BM, lds, wave, X::WAVES, lane);
        return group_count_in(p, c, flag_lds);
    };

    if (wave >= HB + 2) {
        // ---- gather waves
        const int j = wave - (HB + 2);
        const int64_t first = p.block_table ? 0 : (int64_t)c.b * p.L;  // first row of the addressed range
        const char* kv = reinterpret_cast<const char*>(p.kv) + first * 1024;
        const char* kr = reinterpret_cast<const char*>(p.k_rope) + first * 128;
        XsRows rb[X::DEPTH];
#pragma unroll 1
        for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
            for (int i = 0; i < X::DEPTH; ++i) xs_load(p, kv, kr, i, c.nt, idx_lds, j, lane, rb[i]);
            xs_store(X::stage(lds, 0), j, lane, rb[0]);
            xs_load(p, kv, kr, X::DEPTH, c.nt, idx_lds, j, lane, rb[0]);
            xs_store(X::stage(lds, 1), j, lane, rb[1]);
            xs_load(p, kv, kr, X::DEPTH + 1, c.nt, idx_lds, j, lane, rb[1]);
            // Step s: tile s + 2 out of registers into its stage (free since
            // the PV of tile s - 2 in step s - 1), tile s + 5 into the freed
            // registers.  Steps 0 .. nt run in groups of DEPTH (static register
            // indices) with the last partial group outside the loop: an exit
            // inside the loop body would make the compiler's wait counts at
            // the loop head conservative (vmcnt(0) before every store).
            auto step = [&](int s, XsRows& b) __attribute__((always_inline)) {
                lds_barrier();
                xs_store(X::stage(lds, s + 2), j, lane, b);
                xs_load(p, kv, kr, s + 2 + X::DEPTH, c.nt, idx_lds, j, lane, b);
            };
            static_assert(X::DEPTH == 3, "the step groups below assume three register tiles");
            int s0 = 0;
            for (; s0 + 2 <= c.nt; s0 += 3) {
                step(s0, rb[2]);
                step(s0 + 1, rb[0]);
                step(s0 + 2, rb[1]);
            }
            if (s0 <= c.nt) step(s0, rb[2]);
            if (s0 + 1 <= c.nt) step(s0 + 1, rb[0]);
            if (pass == 1 || !vote(false)) break;
        }
        wait_vmcnt<0>();  // the loads past the range
        lds_barrier();    // every wave past its last ring and P read
        lds_barrier();    // l and the maxima published
        finish();
        return;
    }

    if (wave < HB) {
        // ---- QK waves: S^T = K . Q^T for the tile's two 16-row subtiles.
        const int hb = wave;
        float m_ref = -FLT_MAX, m_true = -FLT_MAX, l_run = 0.f;
#pragma unroll 1
        for (int pass = 0; pass < 2; ++pass) {
            l_run = 0.f;
            if (pass == 1) m_ref = m_true;  // pass 1 runs against the exact max
            bool overflow = false;
            for (int s = 0; s <= c.nt; ++s) {
                lds_barrier();
                if (s == c.nt) break;
                const uint32_t stage = X::stage(lds, s);
                // K fragment of k-step ks, subtile sub: row 16 sub + n16, logical
                // chunk 4 ks + qk_lane_chunk(g) (kv) at byte 256 (ks >> 2) +
                // (((4 (ks & 3) + qk_lane_chunk(g)) ^ sw_kv(n16)) << 4); rope chunk
                // 4 (ks - 16) + g at ((4 (ks - 16) + g) ^ sw_rope(n16)) << 4.
                const uint32_t kbase = (stage + n16 * 1024) | ((uint32_t)(qk_lane_chunk(g) ^ sw_kv(n16)) << 4);
                const uint32_t rbase = (stage + X::KV_BYTES + n16 * 128) | ((uint32_t)(g ^ sw_rope(n16)) << 4);
                auto kfrag = [&](int st) -> bf16x8 {
                    const int ks = st >> 1, sub = st & 1;
                    if (ks < 16)
                        return lds_load<bf16x8>((kbase ^ (64u * (ks & 3))) + 256u * (ks >> 2) + sub * 16 * 1024);
                    return lds_load<bf16x8>((rbase ^ (64u * (ks - 16))) + sub * 16 * 128);
                };
                constexpr int KD = XS_QK_DEPTH;
                f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
                i32x4 ivs[2];
                bf16x8 kf[KD];
#pragma unroll
                for (int jj = 0; jj < KD; ++jj) kf[jj] = kfrag(jj);
#pragma unroll
                for (int st = 0; st < 36; ++st) {
                    sacc[st & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[st % KD], qf[st >> 1], sacc[st & 1], 0, 0, 0);
                    if (st + KD < 36) kf[st % KD] = kfrag(st + KD);
                    if (st == 30)
#pragma unroll
                        for (int sub = 0; sub < 2; ++sub)
                            ivs[sub] = lds_load<i32x4>(idx_lds + 4 * (s * BN + 16 * sub + 4 * g));
                    __builtin_amdgcn_sched_barrier(0);
                }
                // Lane holds rows 16 sub + 4 g + r of head n16.  Raw scores with
                // masked rows at -inf; the scale folds into the max and one FMA.
                float x[8];
                float smax = -INFINITY;
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    x[r] = ivs[r >> 2][r & 3] < 0 ? -INFINITY : sacc[r >> 2][r & 3];
                    smax = fmaxf(smax, x[r]);
                }
                smax = max_xor32(max_xor16(smax));
                m_true = fmaxf(m_true, smax * p.score_scale_log2);
                if (m_ref == -FLT_MAX) m_ref = m_true;  // first valid rows: O and l are still zero
                const bool ovf = m_true > m_ref + kRestartLog2;
                overflow |= ovf;
                const float neg_ref = -m_ref;
                float psum = 0.f;
                bf16x8 pk;
                if (__any(ovf)) {  // this pass is to be discarded: the clamp keeps it free of inf
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const float e = fast_exp2(fminf(fmaf(x[r], p.score_scale_log2, neg_ref), kRestartLog2));
                        psum += e;
                        pk[r] = (__bf16)e;
                    }
                } else {  // every P <= 2^kRestartLog2
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const float e = fast_exp2(fmaf(x[r], p.score_scale_log2, neg_ref));
                        psum += e;
                        pk[r] = (__bf16)e;
                    }
                }
                l_run += psum;
                lds_store<bf16x8>(p_lds + (uint32_t)(s & 1) * X::P_BYTES + pp_pchunk(16 * hb + n16, g), pk);
            }
            if (pass == 1 || !vote(overflow)) break;
        }
        lds_barrier();  // every wave past its last ring and P read
        l_run = sum_xor32(sum_xor16(l_run));
        if (g == 0) {
            lds_store<float>(epi + 4 * (16 * hb + n16), l_run);
            lds_store<float>(epi + 4 * (BM + 16 * hb + n16), m_ref);
            lds_store<float>(epi + 4 * (2 * BM + 16 * hb + n16), m_true);
        }
        lds_barrier();  // l and the maxima published
        finish();
        return;
    }

    // ---- PV waves: O^T[columns 256 v ..][heads] += V^T . P^T over each tile's 32 rows
    const int v = wave - HB;
    f32x4 oacc[HB][16];
    // V^T fragment of column block cb: transposed reads of rows 4 g + n16 / 4
    // and 16 + 4 g + n16 / 4 at column 4 (n16 & 3) of the block, i.e. logical
    // chunk 32 v + 2 cb + ((n16 & 3) >> 1), byte 8 (n16 & 1); the row is 1 KiB
    // aligned and (2 cb + c) ^ sw = 2 cb ^ (c ^ sw) for c < 2.
    const int tr_row = 4 * g + (n16 >> 2);
    const uint32_t v_row = (uint32_t)tr_row * 1024 + ((uint32_t)v << 9);
    const uint32_t v_sw = (uint32_t)(((((n16 & 3) >> 1) ^ sw_kv(tr_row)) << 4) + ((n16 & 1) << 3));
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int hb = 0; hb < HB; ++hb)
#pragma unroll
            for (int cb = 0; cb < 16; ++cb) oacc[hb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s <= c.nt; ++s) {
            lds_barrier();
            if (s == 0) continue;
            const int t = s - 1;
            const uint32_t vbase = (X::stage(lds, t) + v_row) | v_sw;
            bf16x8 pf[HB];
#pragma unroll
            for (int hb = 0; hb < HB; ++hb)
                pf[hb] = lds_load<bf16x8>(p_lds + (uint32_t)(t & 1) * X::P_BYTES + pp_pchunk(16 * hb + n16, g));
            auto vfrag = [&](int cb) -> bf16x8 {
                const uint32_t a = vbase ^ (32u * cb);
                const bf16x4 v0 = lds_load_tr(a);
                const bf16x4 v1 = lds_load_tr(a + 16 * 1024);
                return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
            };
            constexpr int PV_DEPTH = XS_PV_DEPTH;
            bf16x8 vf[PV_DEPTH];
#pragma unroll
            for (int jj = 0; jj < PV_DEPTH; ++jj) vf[jj] = vfrag(jj);
#pragma unroll
            for (int cb = 0; cb < 16; ++cb) {
#pragma unroll
                for (int hb = 0; hb < HB; ++hb)
                    oacc[hb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[cb % PV_DEPTH], pf[hb], oacc[hb][cb], 0, 0, 0);
                if (cb + PV_DEPTH < 16) vf[cb % PV_DEPTH] = vfrag(cb + PV_DEPTH);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (pass == 1 || !vote(false)) break;
    }
    lds_barrier();  // every wave past its last ring and P read
    lds_barrier();  // l and the maxima published
    const bool writes_ml = v == 0 && g == 0;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
        const int hl = 16 * hb + n16;
        const float l = lds_load<float>(epi + 4 * hl);
        const float mr = lds_load<float>(epi + 4 * (BM + hl));
        const float mt = lds_load<float>(epi + 4 * (2 * BM + hl));
        const int head = head0 + hl;
        if (p.nsplit == 1) {
            // bf16 rows staged in the ring (a lane holds 4 columns of each of
            // 16 column blocks), stored one 1 KiB head row per instruction.
            const float inv_l = 1.0f / l;  // O and l share m_ref
            const uint32_t srow = lds + (uint32_t)(hl * 1040 + 2 * (256 * v + 4 * g));
#pragma unroll
            for (int cb = 0; cb < 16; ++cb) {
                bf16x4 o;
                o[0] = (__bf16)(oacc[hb][cb][0] * inv_l);
                o[1] = (__bf16)(oacc[hb][cb][1] * inv_l);
                o[2] = (__bf16)(oacc[hb][cb][2] * inv_l);
                o[3] = (__bf16)(oacc[hb][cb][3] * inv_l);
                lds_store<bf16x4>(srow + 32 * cb, o);
            }
            if (writes_ml) {
                p.out_max[(int64_t)c.token * p.H + head] = mt * kLn2;
                p.out_sum[(int64_t)c.token * p.H + head] = l * fast_exp2(mr - mt);
            }
        } else {
            // FP32 rows staged in the ring (finish() stores them); with the
            // in-kernel merge they and m / l are stored agent-coherent for the
            // group's last workgroup (merge_group_cols reads them back).
            const float to_true = fast_exp2(mr - mt);
            const uint32_t srow = lds + (uint32_t)(hl * kPartRow + 4 * (256 * v + 4 * g));
#pragma unroll
            for (int cb = 0; cb < 16; ++cb) lds_store<f32x4>(srow + 64 * cb, oacc[hb][cb] * to_true);
            if (HB > 1 || p.arrivals == nullptr) {
                if (writes_ml) {
                    const int64_t prow = ((int64_t)c.token * p.nsplit + c.sp) * p.H + head;
                    p.part_m[prow] = mt * kLn2;
                    p.part_l[prow] = l * to_true;
                }
            } else if (writes_ml) {
                const int64_t prow = ((int64_t)c.token * p.nsplit + c.sp) * p.H + head;
                __hip_atomic_store(p.part_m + prow, mt * kLn2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(p.part_l + prow, l * to_true, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (finish()) merge_group_cols<16, 2>(p, c, head0, 16, n16, g, v == 0 && g == 0, 16 * v);
}

// ============================================================== ping-pong
// 128 heads per workgroup, 8 waves in two groups of four (wave w is in group
// w / 4; waves w and w + 4 share a SIMD).  Group k owns heads 64k .. 64k+63.
// Per tile a group runs
//   QK + softmax: wave = 16 heads (Q in registers) x the tile's 32 rows; P
//                 (bf16) goes to the group's LDS buffer,
//   PV:           wave = the group's 64 heads x 128 of the 512 columns (O in
//                 registers), P read back from LDS,
// and the two groups run half a tile apart, so that on every SIMD one wave's
// softmax (VALU) overlaps the other wave's MFMAs (a single wave's VALU and
// MFMA instructions do not overlap):
//   half 2t:   group 0 QK + softmax (t)    group 1 PV (t - 1)
//   half 2t+1: group 0 PV (t)              group 1 QK + softmax (t)
// with a workgroup barrier at the start of every half.  Split merge: the
// two-launch path only (no in-kernel merge).
constexpr int kPPWaves = 8;
constexpr int kPPThreads = 64 * kPPWaves;
// K fragments in flight in the QK chain: 7 (with the k-order of
// qk_lane_chunk, C5 -1 % against 6, 5 and 4; 8 spills)
#ifndef PP_QK_DEPTH
#define PP_QK_DEPTH 7
#endif
// Tiles whose gathers are issued before the prologue's full wait (for Q and
// those tiles); the rest of the first three follow it.  1: the first QK
// waits for tile 0 only (C5 -0.2 % against 3, same bits).
#ifndef PP_PRE_TILES
#define PP_PRE_TILES 1
#endif

struct PPLds {
    static constexpr int BN = 32, NSTAGE = 4;
    static constexpr int KV_BYTES = BN * 1024;
    static constexpr int STAGE_BYTES = BN * 1152;
    static constexpr int IDX_OFF = NSTAGE * STAGE_BYTES;
    // P of one group: 64 heads x 32 bf16 in the k order of the PV B operand
    // (position 8 g + j holds tile row 4 g + j for j < 4, 16 + 4 g + j - 4
    // otherwise), 64 bytes per head; the 16-byte chunk of k-group g of head h
    // sits at pp_pchunk(h, g).
    static constexpr int P_OFF = IDX_OFF + DSA_IDX_CAP * 4;
    static constexpr int P_GROUP = 64 * 64;
    static constexpr int LDS_BYTES = P_OFF + 2 * P_GROUP;
    // per group-0 wave and tile: 8 kv rows + 8 rope rows
    static constexpr int LOADS_PER_TILE = 9;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(DSA_IDX_CAP % 256 == 0, "index cache fetched by the first 256 threads");
    __device__ static uint32_t stage(uint32_t lds, int t) { return lds + (uint32_t)(t % NSTAGE) * STAGE_BYTES; }
};


// Gather of tile t, by the four waves of group 0 (gw = wave 0..3): kv rows
// 8 gw .. 8 gw + 7 (one instruction per row) and rope rows 8 gw .. 8 gw + 7
// (one instruction).  Group 1 issues nothing: the gathers are issued in the
// half-steps in which group 0 runs PV, off the critical QK path.
__device__ __forceinline__ void pp_issue(const FwdParams& p, const Gather& gt, int t, uint32_t stage,
                                         uint32_t idx_lds, int gw, int lane) {
    // Lane-dependent addresses from an opaque copy of the lane id: hoisted out
    // of the pass loop they would be spilled, and each reload's vmcnt(0) would
    // wait for the gathers just issued.
    asm volatile("" : "+v"(lane));
    const int rows = p.kv_rows;
    const int r0 = 8 * gw;
    const int my_id = lds_load<int>(idx_lds + 4 * (t * PPLds::BN + r0 + (lane & 7)));
    const uint32_t my_row = (uint32_t)min(max(my_id, 0), rows - 1);
    const uint32_t lane16 = (uint32_t)lane << 4;
#pragma unroll
    for (int rr = 0; rr < 8; ++rr)
        gather_row(stage + (r0 + rr) * 1024, row_rsrc(gt.kv, __builtin_amdgcn_readlane(my_row, rr)), lane16,
                   (uint32_t)sw_kv(r0 + rr) << 4);
    const int r = r0 + (lane >> 3);
    const int id = lds_load<int>(idx_lds + 4 * (t * PPLds::BN + r));
    const uint32_t voff = ((uint32_t)min(max(id, 0), rows - 1) << 7) + (((lane & 7) ^ sw_rope(r)) << 4);
    gather_lanes(stage + PPLds::KV_BYTES + r0 * 128, gt.kr, voff);
}

__global__ __launch_bounds__(kPPThreads, 1) void sparse_mla_fwd_pp(FwdParams p) {
    using X = PPLds;
    constexpr int BN = X::BN;
    __shared__ __attribute__((aligned(1024))) char smem[X::LDS_BYTES];
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave >> 2;  // 0: QK half-steps even, 1: odd
    const int gw = wave & 3;    // QK: head block gw of the group; PV: columns 128 gw ..
    const int g = lane >> 4;
    const int n16 = lane & 15;

    const WgCoords c = wg_coords<BN>(p);
    const int ghead0 = c.hgi * 128 + 64 * grp;  // first head of the group
    const uint32_t idx_lds = lds + X::IDX_OFF;
    const uint32_t p_lds = lds + X::P_OFF + grp * X::P_GROUP;

    // Index loads first (threads 0..255 fill the cache).
    IdxRegs<> ids;
    if (wave < 4) ids = fetch_indices<BN>(p, c);

    // ---- Q fragments of the QK heads: lane holds Q[head][32 ks + 8
    // qk_lane_chunk(g) .. + 7]; ks 16, 17 from q_rope (dims 32 (ks - 16) + 8 g).
    bf16x8 qf[18];
    {
        const int head = ghead0 + 16 * gw + n16;
        const uint16_t* qrow = p.q + ((int64_t)c.token * p.H + head) * 512 + 8 * qk_lane_chunk(g);
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + 32 * ks);
        const uint16_t* rrow = p.q_rope + ((int64_t)c.token * p.H + head) * 64 + 8 * g;
        qf[16] = *reinterpret_cast<const bf16x8*>(rrow);
        qf[17] = *reinterpret_cast<const bf16x8*>(rrow + 32);
    }
    // Masked slots compacted away (compact_count): the workgroup runs
    // nt = ceil(valid / 32) tiles.  The counts live in group 1's P buffer,
    // which is first written after the barrier that ends the prologue.
    const uint32_t counts = lds + X::P_OFF + X::P_GROUP;
    IdxRegs<> masked;
    if (wave < 4) {
        masked = mask_indices<BN>(ids, p, c);
        compact_count(masked, counts);
    }
    lds_barrier();
    const int valid = compact_total<DSA_IDX_CAP>(counts);
    if (wave < 4) compact_store<BN>(masked, counts, idx_lds, valid);
    const int nt = __builtin_amdgcn_readfirstlane((valid + BN - 1) / BN);
    lds_barrier();
    const Gather gt = make_gather(p, c.b);

    // ---- running state (log2 units) of the 16 QK heads, and O of the PV block
    f32x4 oacc[4][8];  // [head block][column block]
    float m_ref = -FLT_MAX, m_true = -FLT_MAX, l_run = 0.f;

    // This lane's LDS offsets in the tile loop, computed once and held in
    // three registers (made opaque at every use, so that nothing derived from
    // them is hoisted into more registers): off_kv = the K fragment base | the
    // V^T base << 16, both relative to the stage; off_rope = the rope fragment
    // base, relative to the stage; off_p = the P read offset (head block 0;
    // block hb at + 1024 hb, since pp_pchunk's swizzle depends on (h >> 2) & 3
    // = (n16 >> 2) & 3 only) | the P write offset << 16, in the group's P
    // buffer.  Stages are 1 KiB aligned and each base's low bits hold its XOR
    // terms, so stage + base equals the OR of the two.  (Recomputing them from
    // the lane id every half-step took about 45 VALU instructions per tile.)
    uint32_t off_kv, off_rope, off_p;
    {
        const int lg = lane >> 4, ln16 = lane & 15;
        // K fragment of k-step ks, subtile s: row 16 s + n16, logical chunk
        // 4 ks + qk_lane_chunk(g) (kv) at byte 256 (ks >> 2) + (((4 (ks & 3) +
        // qk_lane_chunk(g)) ^ sw_kv(n16)) << 4); rope chunk 4 (ks - 16) + g at
        // ((4 (ks - 16) + g) ^ sw_rope(n16)) << 4.
        const uint32_t koff = (uint32_t)(ln16 * 1024) | ((uint32_t)(qk_lane_chunk(lg) ^ sw_kv(ln16)) << 4);
        // V^T fragment of column block cb (columns 128 gw + 16 cb ..): transposed
        // reads of rows 4 g + n16/4 and 16 + 4 g + n16/4 at column 4 (n16 & 3):
        // logical chunk 16 gw + 2 cb + ((n16 & 3) >> 1), byte 8 (n16 & 1); the
        // row is 1 KiB aligned and (2 cb + c) ^ sw = 2 cb ^ (c ^ sw) for c < 2.
        const int tr_row = 4 * lg + (ln16 >> 2);
        const uint32_t voff = (uint32_t)(tr_row * 1024 + (gw << 8)) +
                              ((uint32_t)((((ln16 & 3) >> 1) ^ sw_kv(tr_row)) << 4) + ((ln16 & 1) << 3));
        off_kv = koff | (voff << 16);
        off_rope = (uint32_t)(X::KV_BYTES + ln16 * 128) | ((uint32_t)(lg ^ sw_rope(ln16)) << 4);
        off_p = pp_pchunk(ln16, lg) | (pp_pchunk(16 * gw + ln16, lg) << 16);
    }
    static_assert(X::KV_BYTES + 16 * 128 <= 0xffff && 32 * 1024 <= 0xffff, "offsets fit 16 bits");

    // QK + softmax of tile t for this wave's 16 heads; P to the group buffer.
    auto qk_softmax = [&](int t, bool& overflow) __attribute__((always_inline)) {
        const uint32_t stage = X::stage(lds, t);
        asm volatile("" : "+v"(off_kv), "+v"(off_rope), "+v"(off_p));
        const uint32_t kbase = stage + (off_kv & 0xffffu);
        const uint32_t rbase = stage + off_rope;
        auto kfrag = [&](int step) -> bf16x8 {
            const int ks = step >> 1, sub = step & 1;
            if (ks < 16) return lds_load<bf16x8>((kbase ^ (64u * (ks & 3))) + 256u * (ks >> 2) + sub * 16 * 1024);
            return lds_load<bf16x8>((rbase ^ (64u * (ks - 16))) + sub * 16 * 128);
        };
        constexpr int KD = PP_QK_DEPTH;
        // The chain is on the critical path of its half-step: it runs at a
        // raised wave priority over the other group's PV.
        __builtin_amdgcn_s_setprio(2);
        f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
        bf16x8 kf[KD];
#pragma unroll
        for (int j = 0; j < KD; ++j) kf[j] = kfrag(j);
#pragma unroll
        for (int step = 0; step < 36; ++step) {
            sacc[step & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[step % KD], qf[step >> 1], sacc[step & 1], 0, 0, 0);
            if (step + KD < 36) kf[step % KD] = kfrag(step + KD);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
        // Lane holds rows 16 s + 4 g + r of head n16.  Raw scores; the
        // compacted slots are all valid except the padding (-1) of the last
        // tile, whose rows are masked at -inf.  The scale folds into the max
        // and one FMA per score.
        float x[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) x[r] = sacc[r >> 2][r & 3];
        if (t == nt - 1) {
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int lg = ln >> 4;
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
                const i32x4 iv = lds_load<i32x4>(idx_lds + 4 * (t * BN + 16 * sub + 4 * lg));
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (iv[r] < 0) x[4 * sub + r] = -INFINITY;
            }
        }
        float smax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 8; ++r) smax = fmaxf(smax, x[r]);
        smax = max_xor32(max_xor16(smax));
        m_true = fmaxf(m_true, smax * p.score_scale_log2);
        if (m_ref == -FLT_MAX) m_ref = m_true;  // first valid rows: O and l are still zero
        const bool ovf = m_true > m_ref + kRestartLog2;
        overflow |= ovf;
        const float neg_ref = -m_ref;
        float psum = 0.f;
        bf16x8 pk;
        if (__any(ovf)) {  // this pass is to be discarded: the clamp keeps it free of inf
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const float e = fast_exp2(fminf(fmaf(x[r], p.score_scale_log2, neg_ref), kRestartLog2));
                psum += e;
                pk[r] = (__bf16)e;
            }
        } else {  // every P <= 2^kRestartLog2
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const float e = fast_exp2(fmaf(x[r], p.score_scale_log2, neg_ref));
                psum += e;
                pk[r] = (__bf16)e;
            }
        }
        l_run += psum;
        lds_store<bf16x8>(p_lds + (off_p >> 16), pk);
    };

    // PV of tile t: O[head block hb][column block cb] += V^T . P^T over the
    // tile's 32 rows (one 16x16x32 MFMA per block pair).
    auto pv = [&](int t) __attribute__((always_inline)) {
        const uint32_t stage = X::stage(lds, t);
        asm volatile("" : "+v"(off_kv), "+v"(off_p));
        bf16x8 pf[4];
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) pf[hb] = lds_load<bf16x8>(p_lds + (off_p & 0xffffu) + 1024 * hb);
        const uint32_t vbase = stage + (off_kv >> 16);
        auto vfrag = [&](int cb) -> bf16x8 {
            const uint32_t a = vbase ^ (32u * cb);
            const bf16x4 v0 = lds_load_tr(a);
            const bf16x4 v1 = lds_load_tr(a + 16 * 1024);
            return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
        };
        bf16x8 vf[2];
        vf[0] = vfrag(0);
        vf[1] = vfrag(1);
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
#pragma unroll
            for (int hb = 0; hb < 4; ++hb)
                oacc[hb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[cb & 1], pf[hb], oacc[hb][cb], 0, 0, 0);
            if (cb + 2 < 8) vf[cb & 1] = vfrag(cb + 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // At most two passes over the range (see kRestartLog2), as in the wide variant.
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int hb = 0; hb < 4; ++hb)
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) oacc[hb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        l_run = 0.f;
        if (pass == 1) m_ref = m_true;
        bool overflow = false;
        if (grp == 0)
#pragma unroll
            for (int i = 0; i < PP_PRE_TILES; ++i)
                if (i < nt) pp_issue(p, gt, i, X::stage(lds, i), idx_lds, gw, lane);
        // Q and the first PP_PRE_TILES tiles complete here (a full wait: the
        // compiler does not count the gathers, see the wide variant); the
        // loop's own waits cover the tiles issued after it.
        wait_vmcnt<0>();
        if (grp == 0)
#pragma unroll
            for (int i = PP_PRE_TILES; i < 3; ++i)
                if (i < nt) pp_issue(p, gt, i, X::stage(lds, i), idx_lds, gw, lane);

        // Half 2t starts when group 0's gathers of tile t have landed (tiles up
        // to t + 2 issued) and every wave is past half 2t - 1; in half 2t + 1
        // group 0 issues tile t + 3 into the stage of tile t - 1, whose last
        // reader (group 1's PV) ran in half 2t.
        if (grp == 0) {
            for (int t = 0; t < nt; ++t) {
                const int ahead = min(2, nt - 1 - t);
                if (ahead >= 2) wait_vmcnt<2 * X::LOADS_PER_TILE>();
                else if (ahead == 1) wait_vmcnt<X::LOADS_PER_TILE>();
                else wait_vmcnt<0>();
                lds_barrier();
                qk_softmax(t, overflow);
                lds_barrier();
                if (t + 3 < nt) pp_issue(p, gt, t + 3, X::stage(lds, t + 3), idx_lds, gw, lane);
                pv(t);
            }
            if (nt > 0) lds_barrier();  // half 2 nt: group 1's last PV
        } else if (nt > 0) {
            lds_barrier();
            lds_barrier();
            qk_softmax(0, overflow);
            for (int t = 1; t < nt; ++t) {
                lds_barrier();
                pv(t - 1);
                lds_barrier();
                qk_softmax(t, overflow);
            }
            lds_barrier();
            pv(nt - 1);
        }
        // ---- workgroup vote: does any head need pass 1?  (The flag lives in
        // the P buffers, free once every wave is past its last PV.)
        if (pass == 1) break;
        const uint32_t flag_lds = lds + X::P_OFF;
        lds_barrier();
        if (threadIdx.x == 0) lds_store<int>(flag_lds, 0);
        lds_barrier();
        if (__any(overflow) && lane == 0) lds_store<int>(flag_lds, 1);
        lds_barrier();
        if (__builtin_amdgcn_readfirstlane(lds_load<int>(flag_lds)) == 0) break;
    }

    // ---- epilogue: the QK waves publish (l, m_ref, m_true) of their heads;
    // the PV waves scale their blocks.  Staging lives in the ring (free).
    lds_barrier();  // every wave is past its last ring and P read
    const uint32_t ml = lds + X::IDX_OFF;  // [3][128] floats (index cache no longer needed)
    l_run = sum_xor32(sum_xor16(l_run));
    int eln = lane;
    asm volatile("" : "+v"(eln));
    const int eg = eln >> 4, en16 = eln & 15;
    if (eg == 0) {
        const int hl = 64 * grp + 16 * gw + en16;  // head within the workgroup
        lds_store<float>(ml + 4 * hl, l_run);
        lds_store<float>(ml + 4 * (128 + hl), m_ref);
        lds_store<float>(ml + 4 * (256 + hl), m_true);
    }
    lds_barrier();
    if (p.nsplit == 1) {
        constexpr int HROW = 1040;  // bytes per staged head row (1 KiB + 16: spreads heads over the banks)
        static_assert(128 * HROW <= X::IDX_OFF, "staged rows fit the ring");
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) {
            const int hl = 64 * grp + 16 * hb + en16;
            const float l = lds_load<float>(ml + 4 * hl);
            const float mr = lds_load<float>(ml + 4 * (128 + hl));
            const float mt = lds_load<float>(ml + 4 * (256 + hl));
            const float inv_l = 1.0f / l;  // O and l share m_ref
            const uint32_t srow = lds + (uint32_t)(hl * HROW + 2 * (128 * gw + 4 * eg));
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) {
                bf16x4 v;
                v[0] = (__bf16)(oacc[hb][cb][0] * inv_l);
                v[1] = (__bf16)(oacc[hb][cb][1] * inv_l);
                v[2] = (__bf16)(oacc[hb][cb][2] * inv_l);
                v[3] = (__bf16)(oacc[hb][cb][3] * inv_l);
                lds_store<bf16x4>(srow + 2 * 16 * cb, v);
            }
            if (gw == 0 && eg == 0) {
                const int head = c.hgi * 128 + hl;
                p.out_max[(int64_t)c.token * p.H + head] = mt * kLn2;
                p.out_sum[(int64_t)c.token * p.H + head] = l * fast_exp2(mr - mt);
            }
        }
        lds_barrier();
        // wave w stores head rows w, w + 8, ...: 64 lanes x 16 bytes = one row
        uint16_t* obase = p.out + ((int64_t)c.token * p.H + c.hgi * 128) * 512 + 8 * eln;
#pragma unroll 4
        for (int hr = wave; hr < 128; hr += kPPWaves)
            *reinterpret_cast<bf16x8*>(obase + (int64_t)hr * 512) = lds_load<bf16x8>(lds + hr * HROW + 16 * eln);
    } else {
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) {
            const int hl = 64 * grp + 16 * hb + en16;
            const int head = c.hgi * 128 + hl;
            const float l = lds_load<float>(ml + 4 * hl);
            const float mr = lds_load<float>(ml + 4 * (128 + hl));
            const float mt = lds_load<float>(ml + 4 * (256 + hl));
            const float to_true = fast_exp2(mr - mt);
            const int64_t prow = ((int64_t)c.token * p.nsplit + c.sp) * p.H + head;
            float* orow = p.part_o + prow * 512 + 128 * gw + 4 * eg;
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) *reinterpret_cast<f32x4*>(orow + 16 * cb) = oacc[hb][cb] * to_true;
            if (gw == 0 && eg == 0) {
                p.part_m[prow] = mt * kLn2;
                p.part_l[prow] = l * to_true;
            }
        }
    }
}

template <typename K>
int launch(K kernel, const FwdParams& p, hipStream_t stream, int threads = kThreads) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)fwd_grid(p)), dim3(threads), 0, stream, p);
    return (int)hipGetLastError();
}


}  // namespace

bool fwd_variant_exists(int hpg, int kvw, int bn, int stages, int mfma, int pv_cols) {
    if (pv_cols == 128 && hpg == 128)  // ping-pong: eight waves, 32-row tiles in a 4-stage ring
        return mfma == 16 && kvw == 1 && bn == 32 && stages == 4;
    if (pv_cols == 128 && (hpg == 16 || hpg == 32) && bn == 32)  // specialised waves: 32-row tiles, 4 stages
        return mfma == 16 && kvw == 2 && stages == 4;
    if (pv_cols == 128)  // column-split PV: four waves, 64-row tiles, 16, 32 or 64 heads
        return mfma == 16 && kvw == 4 && bn == 64 && stages == 2 && (hpg == 16 || hpg == 32 || hpg == 64);
    if (pv_cols != 512) return false;
    if (mfma == 32)
        return (hpg == 128 && kvw == 1 && bn == 32 && stages == 4) || (hpg == 64 && kvw == 2 && bn == 64 && stages == 2);
    if (mfma == 16 && bn == 64 && stages == 2)
        return (hpg == 64 && kvw == 1) || (hpg == 32 && kvw == 2) || (hpg == 16 && kvw == 4);
    return false;
}

int64_t fwd_grid(const FwdParams& p) { return (int64_t)p.rowgroups * p.hgroups; }

int fwd_index_cap(int hpg, int pv_cols) {
    if (pv_cols == 128 && hpg == 64) return XpLds<4>::IDX_CAP;
    return DSA_IDX_CAP;
}

int launch_fwd(const FwdParams& p, int hpg, int kvw, int bn, int stages, int mfma, int pv_cols, hipStream_t stream) {
    if (!fwd_variant_exists(hpg, kvw, bn, stages, mfma, pv_cols)) return (int)hipErrorInvalidValue;
    if (p.kv_fp8 && (mfma != 16 || pv_cols != 512)) return (int)hipErrorInvalidValue;  // fp8 rows: narrow variants only
    if (pv_cols == 128) {
        if (hpg == 128) {
            hipLaunchKernelGGL(sparse_mla_fwd_pp, dim3((unsigned)fwd_grid(p)), dim3(kPPThreads), 0, stream, p);
            return (int)hipGetLastError();
        }
        if (hpg == 16 && bn == 32) return launch(sparse_mla_fwd_xs<1>, p, stream, 64 * XsLds<1>::WAVES);
        if (hpg == 32 && bn == 32) return launch(sparse_mla_fwd_xs<2>, p, stream, 64 * XsLds<2>::WAVES);
        if (hpg == 16) return launch(sparse_mla_fwd_xp<1, true>, p, stream, 2 * kThreads);
        if (hpg == 32) return launch(sparse_mla_fwd_xp<2, false>, p, stream);
        return launch(sparse_mla_fwd_xp<4, false>, p, stream);
    }
    if (mfma == 32) {
        if (hpg == 128) return launch(sparse_mla_fwd_wide<4, 1, 32, 4>, p, stream);
        return launch(sparse_mla_fwd_wide<2, 2, 64, 2>, p, stream);
    }
    if (p.kv_fp8) {
        if (hpg == 64) return launch(sparse_mla_fwd_narrow<4, 1, true>, p, stream);
        if (hpg == 32) return launch(sparse_mla_fwd_narrow<2, 2, true>, p, stream);
        return launch(sparse_mla_fwd_narrow<1, 4, true>, p, stream);
    }
    if (hpg == 64) return launch(sparse_mla_fwd_narrow<4, 1>, p, stream);
    if (hpg == 32) return launch(sparse_mla_fwd_narrow<2, 2>, p, stream);
    return launch(sparse_mla_fwd_narrow<1, 4>, p, stream);
}

}  // namespace dsa
