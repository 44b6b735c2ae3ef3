/*
 * C restatement of the sparse-MLA attention forward.  TEST INFRASTRUCTURE
 * ONLY: loaded by tests/ through oracle/dsa_oracle.py as a checker; the
 * product library never links or calls it.
 *
 * dsa_oracle_exact: FP64 brute force of the operator contract
 *   (FAIRNESS_AUDIT.md:19-26 / tools/review.py:130-145 of the reference):
 *   s_j = (q.kv[I_j] + q_rope.k_rope[I_j]) / 24, -inf for I_j outside [0, L),
 *   m = max s, l = sum exp(s - m), out = sum exp(s - m) kv[I_j] / l.
 *
 * dsa_oracle_tiled: the device-side arithmetic of the reference kernels
 *   (dsa/workspace.py:242-390, dsa/merge.py:1-91): FP32 throughout, slots
 *   processed in tiles of `tile` rows with the online-softmax recurrence
 *   (running max initialised to -FLT_MAX, alpha = exp(m_old - m_new)), the sum
 *   over FP32 exponentials, P rounded to bf16 (round to nearest even) before
 *   P.V, `split` contiguous tile ranges producing (m, l, u) partials that are
 *   merged in FP32.  The output is left in fp32 (before the final bf16 cast).
 *
 * Tensors: q [T,H,512], kv [B,L,512], q_rope [T,H,64], k_rope [B,L,64] as bf16
 * bit patterns; idx [T,TOPK] int32; T = B*SQ tokens, token t in batch t / SQ.
 * Outputs: out [T,H,512], max [T,H], sum [T,H] (double or float).
 * Return: 0, or -1 for invalid sizes.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round an fp32 value to the nearest bf16 value, ties to even (IEEE 754). */
static float round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return x; /* inf / nan unchanged */
    const uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    u &= 0xffff0000u;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static int bad_sizes(int B, int SQ, int H, int L, int K) {
    return B <= 0 || SQ <= 0 || H <= 0 || L <= 0 || K <= 0;
}

int dsa_oracle_exact(const uint16_t* q, const uint16_t* kv, const uint16_t* qr, const uint16_t* kr,
                     const int32_t* idx, int B, int SQ, int H, int L, int K, double* out, double* omax,
                     double* osum) {
    if (bad_sizes(B, SQ, H, L, K)) return -1;
    const int T = B * SQ;
#pragma omp parallel for schedule(dynamic)
    for (int th = 0; th < T * H; ++th) {
        const int t = th / H, h = th % H, b = t / SQ;
        const uint16_t* qv = q + ((size_t)t * H + h) * 512;
        const uint16_t* qrv = qr + ((size_t)t * H + h) * 64;
        double* s = (double*)malloc(sizeof(double) * K);
        double m = -INFINITY;
        for (int j = 0; j < K; ++j) {
            const int id = idx[(size_t)t * K + j];
            if (id < 0 || id >= L) {
                s[j] = -INFINITY;
                continue;
            }
            const uint16_t* kvr = kv + ((size_t)b * L + id) * 512;
            const uint16_t* krr = kr + ((size_t)b * L + id) * 64;
            double acc = 0.0;
            for (int d = 0; d < 512; ++d) acc += (double)bf16_to_f32(qv[d]) * bf16_to_f32(kvr[d]);
            for (int d = 0; d < 64; ++d) acc += (double)bf16_to_f32(qrv[d]) * bf16_to_f32(krr[d]);
            s[j] = acc / 24.0;
            if (s[j] > m) m = s[j];
        }
        double l = 0.0;
        double u[512];
        for (int d = 0; d < 512; ++d) u[d] = 0.0;
        for (int j = 0; j < K; ++j) {
            if (s[j] == -INFINITY) continue;
            const double p = exp(s[j] - m);
            l += p;
            const uint16_t* kvr = kv + ((size_t)b * L + idx[(size_t)t * K + j]) * 512;
            for (int d = 0; d < 512; ++d) u[d] += p * bf16_to_f32(kvr[d]);
        }
        for (int d = 0; d < 512; ++d) out[((size_t)t * H + h) * 512 + d] = u[d] / l;
        omax[(size_t)t * H + h] = m;
        osum[(size_t)t * H + h] = l;
        free(s);
    }
    return 0;
}

int dsa_oracle_tiled(const uint16_t* q, const uint16_t* kv, const uint16_t* qr, const uint16_t* kr,
                     const int32_t* idx, int B, int SQ, int H, int L, int K, int tile, int split, float* out,
                     float* omax, float* osum) {
    if (bad_sizes(B, SQ, H, L, K) || tile <= 0 || split <= 0) return -1;
    const int T = B * SQ;
    const int ntiles = (K + tile - 1) / tile;
    if (split > ntiles) return -1;
    const float scale = 1.0f / 24.0f;
#pragma omp parallel for schedule(dynamic)
    for (int th = 0; th < T * H; ++th) {
        const int t = th / H, h = th % H, b = t / SQ;
        const uint16_t* qv = q + ((size_t)t * H + h) * 512;
        const uint16_t* qrv = qr + ((size_t)t * H + h) * 64;
        float* pm = (float*)malloc(sizeof(float) * split);
        float* pl = (float*)malloc(sizeof(float) * split);
        float* pu = (float*)malloc(sizeof(float) * split * 512);
        float* x = (float*)malloc(sizeof(float) * tile);
        for (int sp = 0; sp < split; ++sp) {
            float m = -FLT_MAX, l = 0.f;
            float* u = pu + (size_t)sp * 512;
            for (int d = 0; d < 512; ++d) u[d] = 0.f;
            const int tb = (int)((long)sp * ntiles / split), te = (int)((long)(sp + 1) * ntiles / split);
            for (int tt = tb; tt < te; ++tt) {
                float mt = -INFINITY;
                for (int r = 0; r < tile; ++r) {
                    const int slot = tt * tile + r;
                    const int id = slot < K ? idx[(size_t)t * K + slot] : -1;
                    if (id < 0 || id >= L) {
                        x[r] = -INFINITY;
                        continue;
                    }
                    const uint16_t* kvr = kv + ((size_t)b * L + id) * 512;
                    const uint16_t* krr = kr + ((size_t)b * L + id) * 64;
                    float acc = 0.f;
                    for (int d = 0; d < 512; ++d) acc += bf16_to_f32(qv[d]) * bf16_to_f32(kvr[d]);
                    for (int d = 0; d < 64; ++d) acc += bf16_to_f32(qrv[d]) * bf16_to_f32(krr[d]);
                    x[r] = acc * scale;
                    if (x[r] > mt) mt = x[r];
                }
                const float mn = mt > m ? mt : m;
                const float alpha = expf(m - mn);
                float ps = 0.f;
                for (int d = 0; d < 512; ++d) u[d] *= alpha;
                for (int r = 0; r < tile; ++r) {
                    const float p = expf(x[r] - mn);
                    ps += p;
                    if (p == 0.f) continue;
                    const float pb = round_bf16(p);
                    const int id = idx[(size_t)t * K + tt * tile + r];
                    const uint16_t* kvr = kv + ((size_t)b * L + id) * 512;
                    for (int d = 0; d < 512; ++d) u[d] += pb * bf16_to_f32(kvr[d]);
                }
                l = alpha * l + ps;
                m = mn;
            }
            pm[sp] = m;
            pl[sp] = l;
        }
        float mm = -FLT_MAX;
        for (int sp = 0; sp < split; ++sp) mm = pm[sp] > mm ? pm[sp] : mm;
        float ll = 0.f;
        float uu[512];
        for (int d = 0; d < 512; ++d) uu[d] = 0.f;
        for (int sp = 0; sp < split; ++sp) {
            const float w = expf(pm[sp] - mm);
            ll += w * pl[sp];
            for (int d = 0; d < 512; ++d) uu[d] += w * pu[(size_t)sp * 512 + d];
        }
        for (int d = 0; d < 512; ++d) out[((size_t)t * H + h) * 512 + d] = uu[d] / ll;
        omax[(size_t)t * H + h] = mm;
        osum[(size_t)t * H + h] = ll;
        free(pm);
        free(pl);
        free(pu);
        free(x);
    }
    return 0;
}
