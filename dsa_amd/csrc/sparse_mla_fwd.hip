// Sparse-MLA attention forward for gfx950 (MI355X).
//
// One workgroup owns (token, KV split, head group).  It gathers the selected
// 576-wide rows (kv[:512] ++ k_rope[:64]) straight from HBM into an LDS ring
// with global_load_lds_dwordx4 (no VGPR staging), and every wave computes, for
// its 16 heads,
//
//   S^T[row, head] = K[row, :576] . Q[head, :576]      (v_mfma_f32_16x16x32_bf16,
//                                                       A = K from LDS, B = Q in VGPRs)
//   online softmax over rows in registers (log2 units, FP32 state)
//   O^T[col, head] += V^T[col, row] . P^T[row, head]   (A = V read with
//                                                       ds_read_b64_tr_b16, B = P in VGPRs)
//
// S^T puts the head on lane & 15, which is exactly the lane layout the PV
// B operand needs, so P never leaves registers.  All heads of the group share
// one gathered tile.
//
// Math follows the reference workspace kernel (dsa/workspace.py:242-390):
// running max initialised to -FLT_MAX (:68), scores scaled and masked by the
// raw index (:252-257), alpha = exp(m_old - m_new), FP32 sum of the FP32
// exponentials, P rounded to bf16 (RNE) before PV (:270-272), FP32 accumulation,
// and for split > 1 the unnormalised FP32 numerator plus (max, sum) partials
// (:379-385).  Scores are carried in log2 units (x * log2(e)/24) so that every
// exponential is one v_exp_f32; max/sum leave the kernel in natural units.
#include <hip/hip_runtime.h>
#include <float.h>
#include <stdint.h>

#include "kernels.h"
#include "../../include/dsa_mi355x.h"

namespace dsa {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;

// log2(e) / 24: multiplying the raw QK dot product by this gives the score in
// log2 units, so exp(score - max) == exp2(x - x_max).
constexpr float kScoreLog2 = (float)(1.4426950408889634 / 24.0);
constexpr float kLn2 = 0.69314718055994531f;

// ---------------------------------------------------------------- LDS access
// LDS is addressed through 32-bit byte addresses in address space 3.
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

// Gather one 16-byte chunk per lane from global memory into LDS at
// m0 + 16 * lane.  Issued as inline asm so the compiler does not serialise
// later LDS reads behind it; completion is tracked with wait_vmcnt().
__device__ __forceinline__ void gather16(uint32_t lds_wave_base, const void* gaddr) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds_wave_base), "v"(gaddr)
                 : "memory", "m0");
#pragma clang diagnostic pop
}

// 16-byte chunk swizzles.  A kv row occupies 1024 contiguous LDS bytes (64
// chunks); logical chunk c of tile row r lives at physical chunk c ^ sw_kv(r).
// A rope row occupies 128 bytes (8 chunks): physical = c ^ sw_rope(r).  The
// swizzles make both the QK reads (16 rows x 16 B per quarter-wave) and the
// transposed PV reads (8 rows x 32 B per half-wave) bank-conflict free.
__device__ __forceinline__ int sw_kv(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }
__device__ __forceinline__ int sw_rope(int r) { return (r >> 1) & 7; }

__device__ __forceinline__ float wave_max_over_groups(float v) {
    // lanes l, l^16, l^32, l^48 hold the same head
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}
__device__ __forceinline__ float wave_sum_over_groups(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Store 4 consecutive outputs of one head row: bf16 (final) or fp32 (partial).
__device__ __forceinline__ void store_out4(uint16_t* dst, f32x4 v, float inv_l) {
    bf16x4 b;
    b[0] = (__bf16)(v[0] * inv_l);
    b[1] = (__bf16)(v[1] * inv_l);
    b[2] = (__bf16)(v[2] * inv_l);
    b[3] = (__bf16)(v[3] * inv_l);
    *reinterpret_cast<bf16x4*>(dst) = b;
}

template <int HW, int KW, int BN, int NSTAGE>
struct Layout {
    static constexpr int NW = HW * KW;             // waves per workgroup
    static constexpr int NT = NW * 64;             // threads
    static constexpr int RPW = BN / KW;            // tile rows per wave
    static constexpr int NSUB = RPW / 16;          // 16-row subtiles per wave
    static constexpr int KV_BYTES = BN * 1024;
    static constexpr int ROPE_BYTES = BN * 128;
    static constexpr int STAGE_BYTES = KV_BYTES + ROPE_BYTES;
    static constexpr int IDX_OFF = NSTAGE * STAGE_BYTES;
    static constexpr int LDS_BYTES = IDX_OFF + DSA_IDX_CAP * 4;
    static constexpr int KV_PER_WAVE = BN / NW;    // kv row gathers per wave per tile
    static constexpr int ROPE_PER_WAVE = BN / 8 / NW;  // rope gathers (8 rows each)
    static constexpr int LOADS_PER_TILE = KV_PER_WAVE + ROPE_PER_WAVE;
    // epilogue exchange for KW > 1 (reuses the ring)
    static constexpr int OX_STRIDE = 516;          // floats per head row (padded)
    static constexpr int OX_BYTES = NW * 16 * OX_STRIDE * 4;
    static_assert(BN % (8 * NW) == 0, "rope gathers must split evenly over waves");
    static_assert(RPW == 16 || RPW == 32 || RPW == 64, "rows per wave");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(KW == 1 || OX_BYTES <= IDX_OFF, "epilogue exchange fits the ring");
    static_assert(NSTAGE == 2, "ring depth");
};

template <int HW, int KW, int BN, int NSTAGE>
__global__ __launch_bounds__(HW * KW * 64, 1) void sparse_mla_fwd_kernel(FwdParams p) {
    using C = Layout<HW, KW, BN, NSTAGE>;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hw = wave % HW;
    const int kw = wave / HW;
    const int g = lane >> 4;
    const int n16 = lane & 15;

    // ---- workgroup -> (row group = token * nsplit + split, head group).
    // Workgroups are dispatched round-robin over the 8 XCDs; when possible all
    // head groups of one row group land on the same XCD so the gathered rows
    // are fetched from HBM once and re-read from that XCD's L2.
    const int wg = blockIdx.x;
    int rg, hgi;
    if ((p.rowgroups & 7) == 0) {
        const int j = wg >> 3;
        rg = (wg & 7) + 8 * (j / p.hgroups);
        hgi = j % p.hgroups;
    } else {
        rg = wg / p.hgroups;
        hgi = wg % p.hgroups;
    }
    const int token = rg / p.nsplit;
    const int sp = rg % p.nsplit;
    const int b = token / p.SQ;
    const int head = hgi * (16 * HW) + hw * 16 + n16;  // this lane's head
    const int t_begin = (int)(((int64_t)sp * p.ntiles) / p.nsplit);
    const int t_end = (int)(((int64_t)(sp + 1) * p.ntiles) / p.nsplit);
    const int nt = t_end - t_begin;
    const int slot0 = t_begin * BN;
    const int nslots = nt * BN;  // <= DSA_IDX_CAP, checked on the host
    const int L = p.L;

    // ---- Q fragments: B operand of S^T = K . Q^T.  Lane holds
    // Q[head][32*ks + 8*g .. +7]; ks 16, 17 come from q_rope.
    bf16x8 qf[18];
    {
        const uint16_t* qrow = p.q + ((int64_t)token * p.H + head) * 512 + 8 * g;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + 32 * ks);
        const uint16_t* rrow = p.q_rope + ((int64_t)token * p.H + head) * 64 + 8 * g;
        qf[16] = *reinterpret_cast<const bf16x8*>(rrow);
        qf[17] = *reinterpret_cast<const bf16x8*>(rrow + 32);
    }

    // ---- indices of this workgroup's slot range -> LDS, padded with -1 so a
    // ragged last tile is masked.
    const uint32_t idx_lds = lds + C::IDX_OFF;
    {
        const int32_t* gidx = p.idx + (int64_t)token * p.TOPK;
        for (int s = threadIdx.x; s < nslots; s += C::NT) {
            const int slot = slot0 + s;
            lds_store<int>(idx_lds + 4 * s, slot < p.TOPK ? gidx[slot] : -1);
        }
    }
    lds_barrier();

    const int64_t kv_batch = (int64_t)b * L;
    const char* kv_base = reinterpret_cast<const char*>(p.kv);
    const char* kr_base = reinterpret_cast<const char*>(p.k_rope);

    // ---- gather of tile t (workgroup-local index) into ring stage st.
    auto issue_tile = [&](int t, int st) {
        const uint32_t stage = lds + st * C::STAGE_BYTES;
        const int r0 = wave * C::KV_PER_WAVE;
        const int my_id = lds_load<int>(idx_lds + 4 * (t * BN + r0 + (lane % C::KV_PER_WAVE)));
#pragma unroll
        for (int rr = 0; rr < C::KV_PER_WAVE; ++rr) {
            const int r = r0 + rr;
            int id = __builtin_amdgcn_readlane(my_id, rr);
            id = min(max(id, 0), L - 1);  // address clamp; the mask uses the raw index
            const char* src = kv_base + ((kv_batch + id) << 10) + ((lane ^ sw_kv(r)) << 4);
            gather16(stage + r * 1024, src);
        }
#pragma unroll
        for (int jj = 0; jj < C::ROPE_PER_WAVE; ++jj) {
            const int j = wave * C::ROPE_PER_WAVE + jj;
            const int r = j * 8 + (lane >> 3);
            int id = lds_load<int>(idx_lds + 4 * (t * BN + r));
            id = min(max(id, 0), L - 1);
            const char* src = kr_base + ((kv_batch + id) << 7) + (((lane & 7) ^ sw_rope(r)) << 4);
            gather16(stage + C::KV_BYTES + j * 1024, src);
        }
    };

    // ---- per-lane LDS offsets.  The swizzles depend only on the row mod 16,
    // and XOR-ing a chunk index only touches its low 4 bits, so every fragment
    // address is a per-lane base plus a compile-time multiple of 256 bytes.
    const int rowbase = kw * C::RPW;
    // QK A operand: row rowbase + 16*s + n16, logical chunk 4*ks + g = 16*(ks>>2) + (4*(ks&3) + g)
    uint32_t qk_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) qk_off[j] = ((4 * j + g) ^ sw_kv(n16)) << 4;
    uint32_t rp_off[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) rp_off[j] = ((4 * j + g) ^ sw_rope(n16)) << 4;
    // PV A operand (transposed read): row rowbase + 32*k + 16*h + 4*g + n16/4,
    // column 16*cb + 4*(n16 & 3) -> logical chunk 2*cb + ((n16 & 3) >> 1) =
    // 16*(cb>>3) + (2*(cb&7) + ((n16 & 3) >> 1)), byte 8*(n16 & 1) within it.
    const int tr_row = 4 * g + (n16 >> 2);
    uint32_t tr_off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) tr_off[j] = (((2 * j + ((n16 & 3) >> 1)) ^ sw_kv(tr_row)) << 4) + ((n16 & 1) << 3);

    // ---- running state (log2 units).  P is formed against a reference max
    // m_ref that only moves when the true running max exceeds it by more than
    // kRescaleLog2 (then O and l are rescaled); m_true is the exact running
    // max reported to the caller.  P <= 2^kRescaleLog2, so bf16 P keeps its
    // relative precision and nothing overflows.
    constexpr float kRescaleLog2 = 8.0f;
    f32x4 oacc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_ref = -FLT_MAX;
    float m_true = -FLT_MAX;
    float l_run = 0.f;  // per-lane partial of the head's sum, relative to m_ref

    if (nt > 0) issue_tile(0, 0);

    for (int t = 0; t < nt; ++t) {
        const int st = t & 1;
        wait_vmcnt<0>();
        lds_barrier();
        if (t + 1 < nt) issue_tile(t + 1, st ^ 1);

        const uint32_t stage = lds + st * C::STAGE_BYTES;
        // ---- S^T = K . Q^T for this wave's rows
        f32x4 sacc[C::NSUB];
#pragma unroll
        for (int s = 0; s < C::NSUB; ++s) {
            sacc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
            const uint32_t rowa = stage + (rowbase + 16 * s + n16) * 1024;
#pragma unroll
            for (int ks = 0; ks < 16; ++ks) {
                const bf16x8 a = lds_load<bf16x8>(rowa + qk_off[ks & 3] + ((ks >> 2) << 8));
                sacc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[ks], sacc[s], 0, 0, 0);
            }
            const uint32_t rowr = stage + C::KV_BYTES + (rowbase + 16 * s + n16) * 128;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const bf16x8 a = lds_load<bf16x8>(rowr + rp_off[ks]);
                sacc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[16 + ks], sacc[s], 0, 0, 0);
            }
            // keep the scheduler from hoisting the next subtile's 18 fragments
            __builtin_amdgcn_sched_barrier(0);
        }

        // ---- scale, mask, online softmax.  Lane holds rows
        // rowbase + 16*s + 4*g + r (r = 0..3) of head n16.
        float x[C::NSUB][4];
        float mloc = -INFINITY;
#pragma unroll
        for (int s = 0; s < C::NSUB; ++s) {
            const i32x4 iv = lds_load<i32x4>(idx_lds + 4 * (t * BN + rowbase + 16 * s + 4 * g));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool valid = (unsigned)iv[r] < (unsigned)L;
                const float v = valid ? sacc[s][r] * kScoreLog2 : -INFINITY;
                x[s][r] = v;
                mloc = fmaxf(mloc, v);
            }
        }
        m_true = fmaxf(m_true, wave_max_over_groups(mloc));
        const bool need = m_true > m_ref + kRescaleLog2;
        if (__any(need)) {
            const float nref = need ? m_true : m_ref;
            const float alpha = fast_exp2(m_ref - nref);
            m_ref = nref;
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < 32; ++i) oacc[i] *= alpha;
        }
        float psum = 0.f;
        bf16x4 pb[C::NSUB];
#pragma unroll
        for (int s = 0; s < C::NSUB; ++s) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = fast_exp2(x[s][r] - m_ref);
                psum += e;
                pb[s][r] = (__bf16)e;
            }
        }
        l_run += psum;

        // ---- O^T += V^T . P^T
        if constexpr (C::NSUB >= 2) {
#pragma unroll
            for (int k = 0; k < C::NSUB / 2; ++k) {
                const bf16x8 pk = __builtin_shufflevector(pb[2 * k], pb[2 * k + 1], 0, 1, 2, 3, 4, 5, 6, 7);
                const uint32_t r0a = stage + (rowbase + 32 * k + tr_row) * 1024;
                const uint32_t r1a = r0a + 16 * 1024;
#pragma unroll
                for (int cb = 0; cb < 32; ++cb) {
                    const uint32_t pc = tr_off[cb & 7] + ((cb >> 3) << 8);
                    const bf16x4 v0 = lds_load_tr(r0a + pc);
                    const bf16x4 v1 = lds_load_tr(r1a + pc);
                    const bf16x8 va = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
                    oacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pk, oacc[cb], 0, 0, 0);
                    if ((cb & 7) == 7) __builtin_amdgcn_sched_barrier(0);
                }
            }
        } else {
            const i16x4 pk = __builtin_bit_cast(i16x4, pb[0]);
            const uint32_t r0a = stage + (rowbase + tr_row) * 1024;
#pragma unroll
            for (int cb = 0; cb < 32; ++cb) {
                const uint32_t pc = tr_off[cb & 7] + ((cb >> 3) << 8);
                const i16x4 va = __builtin_bit_cast(i16x4, lds_load_tr(r0a + pc));
                oacc[cb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pk, oacc[cb], 0, 0, 0);
                if ((cb & 7) == 7) __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // ---- epilogue
    l_run = wave_sum_over_groups(l_run);
    int cb_lo = 0, cb_hi = 32;

    if constexpr (KW > 1) {
        // Merge the KW row-split waves of each head slice through LDS (same
        // FP32 merge as the split merge): M = max m_ref_k, w_k = exp(m_ref_k - M).
        lds_barrier();  // every wave is past its last ring read
        const uint32_t ml = lds + C::IDX_OFF;  // [3][NW][16] floats: m_ref, m_true, l
        if (g == 0) {
            lds_store<float>(ml + 4 * (wave * 16 + n16), m_ref);
            lds_store<float>(ml + 4 * (C::NW * 16 + wave * 16 + n16), m_true);
            lds_store<float>(ml + 4 * (2 * C::NW * 16 + wave * 16 + n16), l_run);
        }
        const uint32_t ox = lds + ((wave * 16 + n16) * C::OX_STRIDE + 4 * g) * 4;
#pragma unroll
        for (int cb = 0; cb < 32; ++cb) lds_store<f32x4>(ox + cb * 64, oacc[cb]);
        lds_barrier();
        float mk[KW], lk[KW];
        float mref = -FLT_MAX, mtrue = -FLT_MAX;
#pragma unroll
        for (int k = 0; k < KW; ++k) {
            const int wk = k * HW + hw;
            mk[k] = lds_load<float>(ml + 4 * (wk * 16 + n16));
            mtrue = fmaxf(mtrue, lds_load<float>(ml + 4 * (C::NW * 16 + wk * 16 + n16)));
            lk[k] = lds_load<float>(ml + 4 * (2 * C::NW * 16 + wk * 16 + n16));
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
                    const f32x4 v =
                        lds_load<f32x4>(lds + ((wk * 16 + n16) * C::OX_STRIDE + 4 * g + cb * 16) * 4);
                    acc += wgt[k] * v;
                }
                oacc[cb] = acc;
            }
        }
    }

    // Re-express (m_ref, l, O) against the true max for the caller.
    const float to_true = fast_exp2(m_ref - m_true);
    const float l_fin = l_run * to_true;
    const float m_fin = m_true;
    const float m_nat = m_fin * kLn2;
    if (p.nsplit == 1) {
        const float inv_l = 1.0f / l_run;  // O and l_run share m_ref
        uint16_t* orow = p.out + ((int64_t)token * p.H + head) * 512 + 4 * g;
#pragma unroll
        for (int cb = 0; cb < 32; ++cb)
            if (cb >= cb_lo && cb < cb_hi) store_out4(orow + 16 * cb, oacc[cb], inv_l);
        if (g == 0 && kw == 0) {
            p.out_max[(int64_t)token * p.H + head] = m_nat;
            p.out_sum[(int64_t)token * p.H + head] = l_fin;
        }
    } else {
        const int64_t prow = ((int64_t)token * p.nsplit + sp) * p.H + head;
        float* orow = p.part_o + prow * 512 + 4 * g;
#pragma unroll
        for (int cb = 0; cb < 32; ++cb)
            if (cb >= cb_lo && cb < cb_hi) *reinterpret_cast<f32x4*>(orow + 16 * cb) = oacc[cb] * to_true;
        if (g == 0 && kw == 0) {
            p.part_m[prow] = m_nat;
            p.part_l[prow] = l_fin;
        }
    }
}

template <int HW, int KW, int BN, int NSTAGE>
int launch_variant(const FwdParams& p, hipStream_t stream) {
    using C = Layout<HW, KW, BN, NSTAGE>;
    const int64_t grid = fwd_grid(p);
    hipLaunchKernelGGL((sparse_mla_fwd_kernel<HW, KW, BN, NSTAGE>), dim3((unsigned)grid), dim3(C::NT), 0,
                       stream, p);
    return (int)hipGetLastError();
}

}  // namespace

bool fwd_variant_exists(int hpg, int kvw, int bn, int stages) {
    if (bn != 64 || stages != 2) return false;
    return (hpg == 64 && kvw == 1) || (hpg == 32 && kvw == 2) || (hpg == 16 && kvw == 4);
}

int64_t fwd_grid(const FwdParams& p) { return (int64_t)p.rowgroups * p.hgroups; }

int launch_fwd(const FwdParams& p, int hpg, int kvw, int bn, int stages, hipStream_t stream) {
    if (bn == 64 && stages == 2) {
        if (hpg == 64 && kvw == 1) return launch_variant<4, 1, 64, 2>(p, stream);
        if (hpg == 32 && kvw == 2) return launch_variant<2, 2, 64, 2>(p, stream);
        if (hpg == 16 && kvw == 4) return launch_variant<1, 4, 64, 2>(p, stream);
    }
    return (int)hipErrorInvalidValue;
}

}  // namespace dsa
