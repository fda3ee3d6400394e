// Fused flash attention on gfx950 MFMA (fp16 in, fp32 accumulate / softmax).
//
// Replaces ATTN / ATTN_BIG (attention_f32.comp, attention_big_f32.comp) and the
// SPLIT/MERGE head transposes around them (vk_engine.cpp:649-663): heads are read
// in place from token-major [B*S, ld] buffers at column h*d.
//
// Per wave: 32 queries.  Scores are computed transposed, S^T = K . Q^T, with
// v_mfma_f32_32x32x16_f16 so that lane l owns query l%32 (rows = keys).  The K
// fragment is loaded with a fixed key permutation (swap of key groups 4-7 and
// 8-11 in every 16) so that each lane's score registers are directly the B
// operand of O^T = V^T . P^T, again 32x32x16 with lane l owning query l%32: the
// online-softmax rescale is a per-lane scalar and no cross-lane shuffles are
// needed except one max / sum exchange with lane l^32.  V is staged transposed
// in LDS ([dim][key]) so the A operand is one 16-byte read.
#include "sdu_internal.h"

namespace sdu {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

static constexpr int KT = 64;        // keys per iteration
static constexpr int VSTR = KT + 8;  // Vt row stride (halves)

__device__ __forceinline__ int key_perm(int r) {
    const int o = r & 15;
    const int po = (o >= 4 && o < 8) ? o + 4 : ((o >= 8 && o < 12) ? o - 4 : o);
    return (r & ~15) | po;
}

// KS: 16-wide k-steps covering d for QK^T; MTD: 32-row dim tiles for PV;
// NWAVE: waves per block (32 queries each; they share the K/V tiles in LDS).
template <int KS, int MTD, int NWAVE>
__global__ __launch_bounds__(NWAVE * 64) void attn_kernel(AttnArgs a) {
    constexpr int KSTR = KS * 16 + 8;  // K row stride (halves)
    constexpr int NTH = NWAVE * 64;
    __shared__ __attribute__((aligned(16))) f16 Ks[2][KT * KSTR];
    __shared__ __attribute__((aligned(16))) f16 Vt[2][MTD * 32 * VSTR];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.y, b = blockIdx.z;
    const int d = a.d, dch = d >> 3;  // 16-byte chunks per row
    const int q0 = blockIdx.x * (NWAVE * 32) + wave * 32;
    const int lrow = lane & 31, hl = lane >> 5, lk = hl * 8;
    const float c = a.scale * 1.4426950408889634f;

    // zero the K padding columns [d, KS*16) of both buffers (never overwritten)
    for (int i = tid; i < 2 * KT; i += NTH) {
        f16* row = &Ks[i / KT][(i % KT) * KSTR];
        for (int x = d; x < KS * 16; ++x) row[x] = (f16)0.f;
    }

    // Q fragment (B operand of S^T = K Q^T): lane holds Q[q0+lrow][ks*16+lk .. +7]
    half8 qf[KS];
    {
        const int q = q0 + lrow;
        const f16* qp = a.q + ((int64_t)b * a.Sq + q) * a.ldq + (int64_t)h * d;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int dd = ks * 16 + lk;
            half8 v = {};
            if (q < a.Sq && dd < d) v = *(const half8*)(qp + dd);
            qf[ks] = v;
        }
    }

    floatx16 o[MTD];
#pragma unroll
    for (int t = 0; t < MTD; ++t) o[t] = floatx16{};
    float m_run = -INFINITY, l_run = 0.f;

    const f16* kbase = a.k + (int64_t)b * a.Sk * a.ldk + (int64_t)h * d;
    const f16* vbase = a.v + (int64_t)b * a.Sk * a.ldv + (int64_t)h * d;
    constexpr int MAXCH = (KT * KS * 2 + NTH - 1) / NTH;  // >= KT*d/8/NTH
    uint4 rk[MAXCH], rv[MAXCH];
    const int nchunk = KT * dch;

    auto load_kv = [&](int kb) {
#pragma unroll
        for (int i = 0; i < MAXCH; ++i) {
            const int cidx = tid + i * NTH;
            uint4 kv = make_uint4(0, 0, 0, 0), vv = kv;
            if (cidx < nchunk) {
                const int key = cidx / dch, dc = cidx - key * dch;
                const int j = kb + key;
                if (j < a.Sk) {
                    kv = *(const uint4*)(kbase + (int64_t)j * a.ldk + dc * 8);
                    vv = *(const uint4*)(vbase + (int64_t)j * a.ldv + dc * 8);
                }
            }
            rk[i] = kv;
            rv[i] = vv;
        }
    };
    auto store_kv = [&](int buf) {
#pragma unroll
        for (int i = 0; i < MAXCH; ++i) {
            const int cidx = tid + i * NTH;
            if (cidx < nchunk) {
                const int key = cidx / dch, dc = cidx - key * dch;
                *(uint4*)&Ks[buf][key * KSTR + dc * 8] = rk[i];
                const f16* vh = (const f16*)&rv[i];
#pragma unroll
                for (int e = 0; e < 8; ++e) Vt[buf][(dc * 8 + e) * VSTR + key] = vh[e];
            }
        }
    };

    const int nt = (a.Sk + KT - 1) / KT;
    load_kv(0);
    __syncthreads();  // padding zeroed before the first K stores land next to it
    store_kv(0);
    __syncthreads();

    for (int it = 0; it < nt; ++it) {
        const int buf = it & 1;
        const int kb = it * KT;
        if (it + 1 < nt) load_kv(kb + KT);

        floatx16 s[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            s[sub] = floatx16{};
            const f16* krow = &Ks[buf][(sub * 32 + key_perm(lrow)) * KSTR + lk];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const half8 kf = *(const half8*)(krow + ks * 16);
                s[sub] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], s[sub], 0, 0, 0);
            }
        }
        // scale into the log2 domain, mask keys >= Sk, tile max
        float mx = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = (e >> 2) * 8 + hl * 4 + (e & 3);
                const int key = kb + sub * 32 + key_perm(r);
                const float v = (key < a.Sk) ? s[sub][e] * c : -INFINITY;
                s[sub][e] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = exp2f(m_run - m_new);  // m_run = -inf on the first tile -> 0
        float psum = 0.f;
        half8 pf[2][2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float p = exp2f(s[sub][st * 8 + i] - m_new);
                    psum += p;
                    pf[sub][st][i] = (f16)p;
                }
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int t = 0; t < MTD; ++t) o[t] *= alpha;
        // O^T += V^T . P^T over the 64 keys (4 k-steps of 16)
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const int kofs = sub * 32 + st * 16 + lk;
#pragma unroll
                for (int t = 0; t < MTD; ++t) {
                    const half8 vf = *(const half8*)&Vt[buf][(t * 32 + lrow) * VSTR + kofs];
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[sub][st], o[t], 0, 0, 0);
                }
            }
        if (it + 1 < nt) store_kv(buf ^ 1);
        __syncthreads();
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = 1.0f / l_tot;
    const int q = q0 + lrow;
    if (q < a.Sq) {
        f16* op = a.o + ((int64_t)b * a.Sq + q) * a.ldo + (int64_t)h * d;
#pragma unroll
        for (int t = 0; t < MTD; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int dim = t * 32 + (e >> 2) * 8 + hl * 4 + (e & 3);
                if (dim < d) op[dim] = (f16)(o[t][e] * inv);
            }
    }
}

// MINNW: the smallest block a head size may use (one-wave blocks at d > 96 would
// need more registers for the K/V prefetch than a wave has).
template <int KS, int MTD, int MINNW>
static void launch_nw(const AttnArgs& a, int nw, hipStream_t s) {
    const dim3 grid4((a.Sq + 127) / 128, a.heads, a.B), grid2((a.Sq + 63) / 64, a.heads, a.B),
        grid1((a.Sq + 31) / 32, a.heads, a.B);
    if (nw < 2 && MINNW > 1) nw = 2;
    char name[32];
    snprintf(name, sizeof name, "attn_kernel<%d,%d,%d>", KS, MTD, nw);
    // algorithmic work: QK^T and PV at the true head size; Q, K, V read and O written once
    const double bh = (double)a.B * a.heads;
    const double flops = 4.0 * bh * a.Sq * a.Sk * a.d;
    const double bytes = 2.0 * bh * a.d * (2.0 * a.Sq + 2.0 * a.Sk);
    launch_timed(name, flops, bytes, [&] {
        if (nw == 4) hipLaunchKernelGGL((attn_kernel<KS, MTD, 4>), grid4, dim3(256), 0, s, a);
        else if (nw == 2) hipLaunchKernelGGL((attn_kernel<KS, MTD, 2>), grid2, dim3(128), 0, s, a);
        else hipLaunchKernelGGL((attn_kernel<KS, MTD, MINNW>), grid1, dim3(64 * MINNW), 0, s, a);
    });
}

hipError_t attention_launch(const AttnArgs& a, hipStream_t s) {
    if (a.d <= 0 || a.d > 160 || (a.d & 7) || a.Sq <= 0 || a.Sk <= 0) return hipErrorInvalidValue;
    // fewer waves per block when the query count alone would not fill the chip
    const int64_t bh = (int64_t)a.heads * a.B;
    int nw = 4;
    if (((a.Sq + 127) / 128) * bh < 512) nw = 2;
    if (nw == 2 && ((a.Sq + 63) / 64) * bh < 512) nw = 1;
    const int d = a.d;
    if (d <= 32) launch_nw<2, 1, 1>(a, nw, s);
    else if (d <= 48) launch_nw<3, 2, 1>(a, nw, s);
    else if (d <= 64) launch_nw<4, 2, 1>(a, nw, s);
    else if (d <= 80) launch_nw<5, 3, 1>(a, nw, s);
    else if (d <= 96) launch_nw<6, 3, 1>(a, nw, s);
    else if (d <= 128) launch_nw<8, 4, 2>(a, nw, s);
    else launch_nw<10, 5, 2>(a, nw, s);
    return hipGetLastError();
}

}  // namespace sdu
