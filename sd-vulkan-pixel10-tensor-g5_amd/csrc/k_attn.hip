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
// needed except one max exchange with lane l^32.  V is staged transposed in LDS
// ([dim][key]) so the A operand is one 16-byte read.
//
// Softmax cost per score: one FMA (scale and max folded), one v_exp_f32, a third
// of a v_max3 and half a packed convert.  The running max is only moved when a
// tile raises it by more than 2^8 (wave-uniform branch), so P = 2^(s*c - m) stays
// <= 256, exact in fp16 and far from overflow, and the O rescale is skipped on
// almost every tile.  When the head size leaves a spare row in the last 32-row
// dim tile, that row of V^T is set to 1 so the PV MFMA also produces the row sums.
// When Q arrives pre-scaled by scale * log2 e (the UNet's query projections fold it
// in) and the head size leaves a spare dimension in the last 16-wide k-step (d = 40),
// the shared-tile kernel also moves the FMA into the MFMA: that dimension of Q holds
// -m against a K column of ones, so the scores come out as s*c - m (ofs_update).
//
// Two kernels:
//   attn_kernel       -- NWAVE query waves share each 64-key K/V tile in LDS
//                        (long sequences: 64x64 self-attention, 4096 tokens);
//   attn_split_kernel -- NSPLIT waves split the keys of one 32-query group and
//                        merge their partial (max, sum, O) through LDS (short query
//                        counts, where one wave per 32 queries cannot fill the chip).
#include "sdu_internal.h"

#include <cstdio>

namespace sdu {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

static constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)
// key-split shared-tile launches: pair counters at the head of the workspace (one per
// query block, head and image; zero between launches), the partial slots after them
static constexpr int kAttnMaxPairs = 16384;
// Shared-tile launches stage V row-major and read it with transposing LDS reads (TRV),
// except with 128-key tiles: per launch, with random operands, d40 at 9216 tokens B=2
// -4.1%, at 4096 tokens B=16 -9%, d80 -10 to -13%, d160 at B=16 -10%, but d40 with
// 128-key tiles (4096 tokens, B=2) +1.5%
static constexpr bool kTRV = true;
static constexpr int kAttnCounterFloats = kAttnMaxPairs;

__device__ __forceinline__ int key_perm(int r) {
    const int o = r & 15;
    const int po = (o >= 4 && o < 8) ? o + 4 : ((o >= 8 && o < 12) ? o - 4 : o);
    return (r & ~15) | po;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// P = 2^x as fp16 for the NSUB 32-key sub-tiles of scores s, x = s * c + nm (MODE 0) or
// s (MODE 1), followed by O^T += V^T . P^T.  Returns the lane's sum of P when the row
// sums do not come from the ones row of V^T (!LSUM).
// V^T fragment (the A operand of O^T += V^T . P^T) for dims t*32 + [0, 32) and keys
// kofs + [0, 16): TR = false reads it from a transposed tile vt [dim][key] (one 16-byte
// read); TR = true from a row-major tile vt [key][dim] with two ds_read_b64_tr_b16, whose
// lane i of each 16-lane group receives element i of 4 consecutive rows: the lane's
// address vlo (tr_lane_offset) selects 4 dims of one key row.
typedef short short4v __attribute__((ext_vector_type(4)));
template <bool TR>
__device__ __forceinline__ half8 vt_frag(const f16* vt, int vstr, int t, int kofs_tile, int lrow, int lk, int vlo) {
    if constexpr (TR) {
        const f16* p = vt + kofs_tile * vstr + t * 32 + vlo;
        const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)p);
        const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) short4v*)(p + 4 * vstr));
        const short r[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        half8 v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __builtin_bit_cast(f16, r[i]);
        return v;
    } else {
        return *(const half8*)&vt[(t * 32 + lrow) * vstr + kofs_tile + lk];
    }
}

// Lane offset (halves) of the transposing reads in a row-major V tile with row stride
// vstr: 16-lane group g takes dims 16 (g % 2) + [0, 16) and keys 8 (g / 2) + [0, 8) of the
// 32x32x16 A operand; its lane j reads key 8 (g / 2) + j / 4 (+ 4 for the second read),
// dims 16 (g % 2) + 4 (j % 4) .. + 3.
__device__ __forceinline__ int tr_lane_offset(int lane, int vstr) {
    const int g = lane >> 4, j = lane & 15;
    return (8 * (g >> 1) + (j >> 2)) * vstr + 16 * (g & 1) + 4 * (j & 3);
}

template <int NSUB, int MTD, bool LSUM, int MODE, bool TR = false>
__device__ __forceinline__ float exp_pv(const floatx16 (&s)[NSUB], float c, float nm, floatx16 (&o)[MTD],
                                        const f16* vt, int vstr, int lrow, int lk, int vlo = 0) {
    float psum = 0.f;
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            half8 pf;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x = s[sub][st * 8 + i];
                const float p = fast_exp2(MODE == 0 ? __builtin_fmaf(x, c, nm) : x);
                if (!LSUM) psum += p;
                pf[i] = (f16)p;
            }
#pragma unroll
            for (int t = 0; t < MTD; ++t) {
                const half8 vf = vt_frag<TR>(vt, vstr, t, sub * 32 + st * 16, lrow, lk, vlo);
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[t], 0, 0, 0);
            }
        }
    return psum;
}

// Scores of keys at or past `kvalid` (tile-relative) to -inf.
template <int NSUB>
__device__ __forceinline__ void mask_tile(floatx16 (&s)[NSUB], int kvalid, int hl) {
    if (kvalid < NSUB * 32) {
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int key = sub * 32 + key_perm((e >> 2) * 8 + hl * 4 + (e & 3));
                if (key >= kvalid) s[sub][e] = -INFINITY;
            }
    }
}

// mask_tile, then the max over the lane's query (both halves of the wave)
template <int NSUB>
__device__ __forceinline__ float mask_max(floatx16 (&s)[NSUB], int kvalid, int hl) {
    mask_tile<NSUB>(s, kvalid, hl);
    float mx = s[0][0];
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[sub][e]);
    return fmaxf(mx, __shfl_xor(mx, 32));
}

// Online-softmax update for NSUB 32-key sub-tiles of raw scores s (S^T layout)
// followed by O^T += V^T . P^T.  `kvalid` = number of valid keys in the tile for this
// lane's query (< NSUB*32 only on the last tile, or below the causal limit; may be <= 0).
// vt: V^T tile [dim][key] with row stride vstr.
template <int NSUB, int MTD, bool LSUM, bool TR = false>
__device__ __forceinline__ void softmax_pv(floatx16 (&s)[NSUB], int kvalid, float c, float& m_run,
                                           float& l_run, floatx16 (&o)[MTD], const f16* vt, int vstr,
                                           int hl, int lrow, int lk, int vlo = 0) {
    const float mxs = mask_max<NSUB>(s, kvalid, hl) * c;
    if (__ballot(mxs > m_run + kRescaleLog2)) {  // wave-uniform
        const float m_new = fmaxf(m_run, mxs);
        const float alpha = fast_exp2(m_run - m_new);  // m_run = -inf on the first tile -> 0
#pragma unroll
        for (int t = 0; t < MTD; ++t) o[t] *= alpha;
        l_run *= alpha;
        m_run = m_new;
    }
    // (a lane whose keys so far were all masked keeps m_run = -inf: subtract 0, so that
    // its masked scores give exp2(-inf) = 0 rather than exp2(-inf + inf))
    const float nm = m_run == -INFINITY ? 0.f : -m_run;
    const float psum = exp_pv<NSUB, MTD, LSUM, 0, TR>(s, c, nm, o, vt, vstr, lrow, lk, vlo);
    if (!LSUM) l_run += psum;
}

// The softmax reference carried inside the MFMA (attn_kernel with OFS): Q holds
// q * scale * log2 e and a spare head dimension holds -m_run against a K column of
// ones, so the scores come out of the QK^T MFMA in log2 units already less the running
// reference m_run, and P = 2^s costs no per-score FMA.  m_run is an fp16 value (the
// type of the dimension that carries it), clamped to +-30000: it is set from the first
// tile and moved whenever a tile's max exceeds it by more than 2^8; P <= 2^8 stays exact
// in fp16 for scores below 30000 + 8 (log2 units).  Masks the tile, rescales O and the
// row sum when the reference moves, and returns true then (wave-uniform): the caller
// rewrites Q's spare dimension and recomputes the tile's scores.
template <int NSUB, int MTD>
__device__ __forceinline__ bool ofs_update(floatx16 (&s)[NSUB], int kvalid, float& m_run, float& l_run,
                                           floatx16 (&o)[MTD], int hl, bool first) {
    const float mx = mask_max<NSUB>(s, kvalid, hl);  // the tile's max less m_run
    if (!__ballot(first || mx > kRescaleLog2)) return false;
    const float m_old = first ? 0.f : m_run;  // the reference the tile's scores carry
    float m_new = m_old + (first ? mx : fmaxf(mx, 0.f));
    m_new = (float)(f16)fminf(fmaxf(m_new, -30000.f), 30000.f);
    const float alpha = first ? 0.f : fast_exp2(m_old - m_new);
#pragma unroll
    for (int t = 0; t < MTD; ++t) o[t] *= alpha;
    l_run *= alpha;
    m_run = m_new;
    return true;
}

// Row sum of P for query lrow at the end: from the ones row of V^T (LSUM: dim
// MTD*32-1 = register 15 of the last dim tile on lanes 32..63) or from the
// per-lane partial sums.
template <int MTD, bool LSUM>
__device__ __forceinline__ float row_sum(const floatx16 (&o)[MTD], float l_run, int lrow) {
    if (LSUM) return __shfl(o[MTD - 1][15], lrow + 32);
    return l_run + __shfl_xor(l_run, 32);
}

// Set rows [d, MTD*32) of a V^T tile of `keys` columns: zero, and the last one to 1
// when LSUM.  Rows below d are written per tile and never touch these.
template <int MTD, bool LSUM>
__device__ __forceinline__ void vt_pad_rows(f16* vt, int vstr, int keys, int d, int tid, int nth) {
    const int rows = MTD * 32 - d;
    for (int i = tid; i < rows * keys; i += nth) {
        const int dim = d + i / keys, key = i % keys;
        vt[dim * vstr + key] = (f16)((LSUM && dim == MTD * 32 - 1) ? 1.f : 0.f);
    }
}

// ----------------------------------------------------------------- shared-tile kernel


// KS: 16-wide k-steps covering d for QK^T; MTD: 32-row dim tiles for PV;
// NWAVE: waves per block (32 queries each; they share the K/V tiles in LDS);
// KT: keys per iteration (64, or 128 for small heads on grids of at most two blocks
// per CU: half the barriers and per-tile softmax overhead per key).
// OFS: Q holds q * scale * log2 e and head dimension d (< KS*16) carries the softmax
// reference (ofs_update): K's column d is 1 and Q's dimension d is -m_run.
// SPL: the keys are split in two parts at a.kpart (a multiple of KT), blockIdx.z = image * 2 +
// part; each part's block stores its unnormalised O^T, reference and row-sum partial into a
// workspace slot, and the pair's second block to finish merges both (see the end).
// TRV: V is staged row-major ([key][dim], 16-byte stores as K) and the PV A operand is
// read with transposing LDS reads (vt_frag) instead of staging V^T.
template <int KS, int MTD, int NWAVE, bool LSUM, int KT = 64, bool OFS = false, bool SPL = false,
          bool TRV = false>
__global__ __launch_bounds__(NWAVE * 64) void attn_kernel(AttnArgs a) {
    // V tile: V^T [dim][key] with row stride KT + 8, or (TRV) V [key][dim] with a row stride
    // of 16 (mod 64) halves: the four key rows one 16-lane transposing read touches then
    // fall on distinct banks
    constexpr int VSTR = TRV ? ((MTD * 32 - 16 + 63) / 64) * 64 + 16 : KT + 8;
    constexpr int VTILE = TRV ? KT * VSTR : MTD * 32 * VSTR;
    constexpr int NSUB = KT / 32;
    constexpr int KSTR = KS * 16 + 8;  // K row stride (halves)
    constexpr int NTH = NWAVE * 64;
    __shared__ __attribute__((aligned(16))) f16 Ks[2][KT * KSTR];
    __shared__ __attribute__((aligned(16))) f16 Vt[2][VTILE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.y;
    const int b = SPL ? (int)(blockIdx.z >> 1) : (int)blockIdx.z, part = SPL ? (int)(blockIdx.z & 1) : 0;
    const int kbeg = part * a.kpart, nkeys = (SPL && part == 0 ? a.kpart : a.Sk) - kbeg;  // this block's keys
    const int d = a.d, dch = d >> 3;  // 16-byte chunks per row
    const int q0 = blockIdx.x * (NWAVE * 32) + wave * 32;
    const int lrow = lane & 31, hl = lane >> 5, lk = hl * 8;
    const float c = a.q_log2 ? 1.f : a.scale * 1.4426950408889634f;

    // zero the K padding columns [d, KS*16) of both buffers (OFS: column d is 1) and set
    // the V^T pad rows (never overwritten by the tile stores)
    for (int i = tid; i < 2 * KT; i += NTH) {
        f16* row = &Ks[i / KT][(i % KT) * KSTR];
        for (int x = d; x < KS * 16; ++x) row[x] = (f16)((OFS && x == d) ? 1.f : 0.f);
    }
    if constexpr (TRV) {
        // dims [d, MTD*32) of every key row: zero, the last one 1 when LSUM (row sums)
        const int pad = MTD * 32 - d;
        for (int i = tid; i < 2 * KT * pad; i += NTH) {
            const int bf = i / (KT * pad), r = i % (KT * pad), key = r / pad, dim = d + r % pad;
            Vt[bf][key * VSTR + dim] = (f16)((LSUM && dim == MTD * 32 - 1) ? 1.f : 0.f);
        }
    } else {
        vt_pad_rows<MTD, LSUM>(Vt[0], VSTR, KT, d, tid, NTH);
        vt_pad_rows<MTD, LSUM>(Vt[1], VSTR, KT, d, tid, NTH);
    }
    const int vlo = TRV ? tr_lane_offset(lane, VSTR) : 0;

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

    // K / V tile loads: buffer loads whose per-thread byte offsets are fixed (tile key
    // 0) and move by one add per tile; keys past Sk and threads without a chunk read
    // past the resource's range and get zeros.  No branches, so all loads of a tile
    // stay in flight while the current tile is computed.
    const f16* kbase = a.k + ((int64_t)b * a.Sk + kbeg) * a.ldk + (int64_t)h * d;
    const f16* vbase = a.v + ((int64_t)b * a.Sk + kbeg) * a.ldv + (int64_t)h * d;
    const __amdgpu_buffer_rsrc_t rsk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)kbase, (short)0, ((nkeys - 1) * a.ldk + d) * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)vbase, (short)0, ((nkeys - 1) * a.ldv + d) * 2, 0x00020000);
    // K: one 16-byte chunk (8 dims of one key) per thread and step, stored as is.
    // V: one unit = the same 8 dims of 4 consecutive keys per thread and step, so that
    // the transposed store to V^T [dim][key] is 8 ds_write_b64 (4 keys of one dim each)
    // instead of 32 two-byte stores.
    constexpr int MAXCH = (KT * KS * 2 + NTH - 1) / NTH;        // >= KT*d/8/NTH
    // V per thread and step: TRV, MAXCH 16-byte chunks (as K); else MAXU units of 4 keys
    constexpr int MAXU = TRV ? MAXCH : (KT / 4 * KS * 2 + NTH - 1) / NTH;  // >= (KT/4)*(d/8)/NTH
    constexpr int VLD = TRV ? 1 : 4;                            // 16-byte loads per unit
    uint4 rk[MAXCH], rv[MAXU][VLD];
    const int nchunk = KT * dch, nunit = KT / 4 * dch;
    uint32_t kvo[MAXCH], vvo[MAXU];
    int sto[MAXCH];  // LDS position of the K chunk: key << 16 | dc*8; -1: no chunk
    int vto[MAXU];   // V unit: first key << 16 | dc*8; -1: no unit
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
        const int cidx = tid + i * NTH;
        const int key = cidx / dch, dc = cidx - key * dch;
        const bool ok = cidx < nchunk;
        kvo[i] = ok ? (uint32_t)((key * a.ldk + dc * 8) * 2) : 0x80000000u;
        sto[i] = ok ? key * 65536 + dc * 8 : -1;
    }
#pragma unroll
    for (int i = 0; i < MAXU; ++i) {
        const int u = tid + i * NTH;
        if constexpr (TRV) {
            const int key = u / dch, dc = u - key * dch;
            const bool ok = u < nchunk;
            vvo[i] = ok ? (uint32_t)((key * a.ldv + dc * 8) * 2) : 0x80000000u;
            vto[i] = ok ? key * VSTR + dc * 8 : -1;  // LDS offset (halves)
        } else {
            const int kq = u / dch, dc = u - kq * dch;
            const bool ok = u < nunit;
            vvo[i] = ok ? (uint32_t)((4 * kq * a.ldv + dc * 8) * 2) : 0x80000000u;
            vto[i] = ok ? 4 * kq * 65536 + dc * 8 : -1;
        }
    }
    auto load_kv = [&](int kb) {
        const uint32_t ko = (uint32_t)(kb * a.ldk * 2), vo = (uint32_t)(kb * a.ldv * 2);
        const uint32_t vrow = (uint32_t)(a.ldv * 2);
#pragma unroll
        for (int i = 0; i < MAXCH; ++i)
            rk[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsk, kvo[i] + ko, 0, 0));
#pragma unroll
        for (int i = 0; i < MAXU; ++i)
#pragma unroll
            for (int j = 0; j < VLD; ++j)
                rv[i][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         rsv, vvo[i] + vo + j * vrow, 0, 0));
    };
    auto store_kv = [&](int buf) {
#pragma unroll
        for (int i = 0; i < MAXCH; ++i)
            if (sto[i] >= 0) *(uint4*)&Ks[buf][(sto[i] >> 16) * KSTR + (sto[i] & 0xffff)] = rk[i];
#pragma unroll
        for (int i = 0; i < MAXU; ++i) {
            if constexpr (TRV) {
                if (vto[i] >= 0) *(uint4*)&Vt[buf][vto[i]] = rv[i][0];
            } else if (vto[i] >= 0) {
                const int key = vto[i] >> 16, c8 = vto[i] & 0xffff;
                const uint32_t* w0 = (const uint32_t*)&rv[i][0];
                const uint32_t* w1 = (const uint32_t*)&rv[i][VLD > 1 ? 1 : 0];
                const uint32_t* w2 = (const uint32_t*)&rv[i][VLD > 2 ? 2 : 0];
                const uint32_t* w3 = (const uint32_t*)&rv[i][VLD > 3 ? 3 : 0];
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    // dims 2*e2 (low halves) and 2*e2+1 (high halves) of the 4 keys
                    const uint32_t lo01 = __builtin_amdgcn_perm(w1[e2], w0[e2], 0x05040100u);
                    const uint32_t lo23 = __builtin_amdgcn_perm(w3[e2], w2[e2], 0x05040100u);
                    const uint32_t hi01 = __builtin_amdgcn_perm(w1[e2], w0[e2], 0x07060302u);
                    const uint32_t hi23 = __builtin_amdgcn_perm(w3[e2], w2[e2], 0x07060302u);
                    *(uint2*)&Vt[buf][(c8 + 2 * e2) * VSTR + key] = make_uint2(lo01, lo23);
                    *(uint2*)&Vt[buf][(c8 + 2 * e2 + 1) * VSTR + key] = make_uint2(hi01, hi23);
                }
            }
        }
    };

    const int nt = (nkeys + KT - 1) / KT;
    load_kv(0);
    __syncthreads();  // padding set before the first tile stores land next to it
    store_kv(0);
    __syncthreads();

    for (int it = 0; it < nt; ++it) {
        const int buf = it & 1;
        const int kb = it * KT;
        // wave priority: highest while issuing the next tile's loads, raised through
        // the scores, softmax and PV, normal for the LDS stores and the barrier
        __builtin_amdgcn_s_setprio(2);
        if (it + 1 < nt) load_kv(kb + KT);
        __builtin_amdgcn_s_setprio(1);

        floatx16 s[NSUB];
        auto qk = [&]() {
#pragma unroll
            for (int sub = 0; sub < NSUB; ++sub) {
                s[sub] = floatx16{};
                const f16* krow = &Ks[buf][(sub * 32 + key_perm(lrow)) * KSTR + lk];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const half8 kf = *(const half8*)(krow + ks * 16);
                    s[sub] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], s[sub], 0, 0, 0);
                }
            }
        };
        qk();
        const int kvalid = min(KT, nkeys - kb);
        if constexpr (OFS) {
            if (ofs_update<NSUB, MTD>(s, kvalid, m_run, l_run, o, hl, it == 0)) {
                // Q's dimension d (k-step d / 16, lanes of half (d / 8) & 1, element 0)
                // takes the new reference; the tile's scores are computed again with it
                const f16 nr = (f16)(-m_run);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    if (ks == (d >> 4) && hl == ((d >> 3) & 1)) qf[ks][0] = nr;
                // (K fragments are read from LDS again rather than kept live from the
                // first pass across the softmax of every tile)
                __asm__ volatile("" ::: "memory");
                qk();
                mask_tile<NSUB>(s, kvalid, hl);
            }
            const float psum = exp_pv<NSUB, MTD, LSUM, 1, TRV>(s, 1.f, 0.f, o, Vt[buf], VSTR, lrow, lk, vlo);
            if (!LSUM) l_run += psum;
        } else {
            softmax_pv<NSUB, MTD, LSUM, TRV>(s, kvalid, c, m_run, l_run, o, Vt[buf], VSTR, hl, lrow, lk, vlo);
        }
        __builtin_amdgcn_s_setprio(0);
        if (it + 1 < nt) store_kv(buf ^ 1);
        __syncthreads();
    }

    const float lsum = row_sum<MTD, LSUM>(o, l_run, lrow);
    const float inv = 1.0f / lsum;
    const int q = q0 + lrow;
    if constexpr (SPL) {
        // This part's normalised output O_p (fp32, the head's d dims), its reference m_p
        // and row sum l_p go to the pair's workspace slot; the pair's second block to
        // finish writes (W_0 O_0 + W_1 O_1) / (W_0 + W_1), W_p = l_p 2^(m_p - max m), reading
        // both parts in part order (its own re-read), so the result does not depend on
        // which finished last.  Ordering as in the GEMM's in-kernel split-K sum:
        // device-coherent (sc1) buffer stores, each wave's vmcnt(0) before the block
        // barrier, a device-scope atomic on the pair's counter, the second block's sc1
        // loads only after the barrier that follows its read of the count.  (Normalised
        // values stored like the output path keep the accumulators in one register
        // range through the key loop.)
        constexpr int CPOL_SC1 = 1 << 4;
        constexpr int PW = (MTD * 16 + 2) * 64;  // floats per wave and part: [MTD*16 + 2][64 lanes]
        __shared__ int last_flag;
        const int blk = (b * a.heads + h) * gridDim.x + blockIdx.x;
        const __amdgpu_buffer_rsrc_t rsP = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.ws + kAttnCounterFloats + (int64_t)blk * 2 * NWAVE * PW), (short)0, 2 * NWAVE * PW * 4, 0x00020000);
        const uint32_t vo = (uint32_t)((wave * PW + lane) * 4);
        const int pso = NWAVE * PW * 4;  // bytes per part
#pragma unroll
        for (int t = 0; t < MTD; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int dim = t * 32 + (e >> 2) * 8 + hl * 4 + (e & 3);
                if (dim < d)
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, o[t][e] * inv), rsP,
                                                          vo + (t * 16 + e) * 256, part * pso, CPOL_SC1);
            }
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, m_run), rsP, vo + MTD * 16 * 256,
                                              part * pso, CPOL_SC1);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, lsum), rsP, vo + (MTD * 16 + 1) * 256,
                                              part * pso, CPOL_SC1);
        __builtin_amdgcn_s_waitcnt((0 & 0xF) | (0x7 << 4) | (0x0 << 8));  // vmcnt(0): this wave's stores are done
        __syncthreads();
        if (tid == 0) {
            unsigned* cnt = (unsigned*)a.ws + blk;
            const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = prev == 1u;
            if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next launch
            last_flag = last;
        }
        __syncthreads();
        if (!last_flag) return;
        auto ld = [&](int pp, int j) {
            return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsP, vo + j * 256, pp * pso, CPOL_SC1));
        };
        const float m0 = ld(0, MTD * 16), m1 = ld(1, MTD * 16);
        const float mm = fmaxf(m0, m1);
        const float w0 = ld(0, MTD * 16 + 1) * fast_exp2(m0 - mm), w1 = ld(1, MTD * 16 + 1) * fast_exp2(m1 - mm);
        const float wn = 1.0f / (w0 + w1);
        if (q < a.Sq) {
            f16* op = a.o + ((int64_t)b * a.Sq + q) * a.ldo + (int64_t)h * d;
#pragma unroll
            for (int t = 0; t < MTD; ++t)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int dim = t * 32 + (e >> 2) * 8 + hl * 4 + (e & 3);
                    if (dim < d) op[dim] = (f16)((w0 * ld(0, t * 16 + e) + w1 * ld(1, t * 16 + e)) * wn);
                }
        }
        return;
    }

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

// ----------------------------------------------------------------- key-split kernel

static constexpr int KTS = 32;         // keys per step
static constexpr int VSTRS = KTS + 8;  // per-wave Vt row stride (halves)

template <int MTD, int NSPLIT>
struct SplitSmem {
    // per-wave V tile: V^T [MTD*32][VSTRS], or (TRV) V [KTS][trv_stride(MTD)]
    static constexpr int trv_stride = ((MTD * 32 - 16 + 63) / 64) * 64 + 16;
    static constexpr int vt_elems = kTRV ? KTS * trv_stride : MTD * 32 * VSTRS;
    static constexpr int vt_bytes = NSPLIT * vt_elems * 2;
    static constexpr int comb_bytes = NSPLIT * (MTD * 32 * 32 + 64) * 4;
    static constexpr int bytes = vt_bytes > comb_bytes ? vt_bytes : comb_bytes;
};

// One block = one group of 32 queries of one (image, head); wave w handles key
// tiles w, w+NSPLIT, ...  K fragments come straight from global memory (each lane
// reads 16 contiguous bytes of one key row); V goes through a per-wave transposed
// LDS tile (4 keys of one dim per 8-byte store).  A wave's next tile is loaded into
// registers while the current one is computed.  Within a wave LDS operations
// complete in order, so the per-wave tile needs no block barrier; one barrier
// separates the key loop from the merge.
template <int KS, int MTD, int NSPLIT, bool LSUM>
__global__ __launch_bounds__(NSPLIT * 64) void attn_split_kernel(AttnArgs a) {
    constexpr int NTH = NSPLIT * 64;
    __shared__ __attribute__((aligned(16))) char smem[SplitSmem<MTD, NSPLIT>::bytes];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.y, b = blockIdx.z;
    const int d = a.d, dch = d >> 3;
    const int q0 = blockIdx.x * 32;
    const int lrow = lane & 31, hl = lane >> 5, lk = hl * 8;
    const float c = a.q_log2 ? 1.f : a.scale * 1.4426950408889634f;
    constexpr int VS = kTRV ? SplitSmem<MTD, NSPLIT>::trv_stride : VSTRS;  // V tile row stride
    f16* vt = (f16*)smem + wave * SplitSmem<MTD, NSPLIT>::vt_elems;

    if constexpr (kTRV) {
        // dims [d, MTD*32) of every key row: zero, the last one 1 when LSUM (row sums)
        const int pad = MTD * 32 - d;
        for (int i = lane; i < KTS * pad; i += 64) {
            const int key = i / pad, dim = d + i % pad;
            vt[key * VS + dim] = (f16)((LSUM && dim == MTD * 32 - 1) ? 1.f : 0.f);
        }
    } else {
        vt_pad_rows<MTD, LSUM>(vt, VSTRS, KTS, d, lane, 64);
    }
    const int vlo = kTRV ? tr_lane_offset(lane, VS) : 0;

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
    // V: one unit = the same 8 dims of 4 consecutive keys per lane, so that the
    // transposed store to V^T [dim][key] is 8 ds_write_b64 (4 keys of one dim each)
    // V per lane and tile: (TRV) MAXU 16-byte chunks (8 dims of one key), else MAXU units of
    // the same 8 dims of 4 consecutive keys
    constexpr int MAXU = kTRV ? (KTS * KS * 2 + 63) / 64 : (KTS / 4 * KS * 2 + 63) / 64;
    constexpr int VLD = kTRV ? 1 : 4;
    const int nunit = kTRV ? KTS * dch : KTS / 4 * dch;
    half8 kf[KS];
    uint4 rv[MAXU][VLD];

    auto load = [&](int kb) {
        const int key = kb + key_perm(lrow);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int dd = ks * 16 + lk;
            half8 v = {};
            if (key < a.Sk && dd < d) v = *(const half8*)(kbase + (int64_t)key * a.ldk + dd);
            kf[ks] = v;
        }
#pragma unroll
        for (int i = 0; i < MAXU; ++i) {
            const int u = lane + i * 64;
            const int kq = u / dch, dc = u - kq * dch;
#pragma unroll
            for (int j = 0; j < VLD; ++j) {
                const int key = kb + (kTRV ? kq : 4 * kq + j);
                uint4 vv = make_uint4(0, 0, 0, 0);
                if (u < nunit && key < a.Sk) vv = *(const uint4*)(vbase + (int64_t)key * a.ldv + dc * 8);
                rv[i][j] = vv;
            }
        }
    };
    auto store_v = [&]() {
#pragma unroll
        for (int i = 0; i < MAXU; ++i) {
            const int u = lane + i * 64;
            if (kTRV) {
                const int kq = u / dch;
                if (u < nunit) *(uint4*)&vt[kq * VS + (u - kq * dch) * 8] = rv[i][0];
            } else if (u < nunit) {
                const int kq = u / dch, c8 = (u - kq * dch) * 8, key = 4 * kq;
                const uint32_t* w0 = (const uint32_t*)&rv[i][0];
                const uint32_t* w1 = (const uint32_t*)&rv[i][VLD > 1 ? 1 : 0];
                const uint32_t* w2 = (const uint32_t*)&rv[i][VLD > 2 ? 2 : 0];
                const uint32_t* w3 = (const uint32_t*)&rv[i][VLD > 3 ? 3 : 0];
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    // dims 2*e2 (low halves) and 2*e2+1 (high halves) of the 4 keys
                    const uint32_t lo01 = __builtin_amdgcn_perm(w1[e2], w0[e2], 0x05040100u);
                    const uint32_t lo23 = __builtin_amdgcn_perm(w3[e2], w2[e2], 0x05040100u);
                    const uint32_t hi01 = __builtin_amdgcn_perm(w1[e2], w0[e2], 0x07060302u);
                    const uint32_t hi23 = __builtin_amdgcn_perm(w3[e2], w2[e2], 0x07060302u);
                    *(uint2*)&vt[(c8 + 2 * e2) * VSTRS + key] = make_uint2(lo01, lo23);
                    *(uint2*)&vt[(c8 + 2 * e2 + 1) * VSTRS + key] = make_uint2(hi01, hi23);
                }
            }
        }
    };

    // Each wave's tiles: the next tile's K and V are loaded into registers while the
    // current one's softmax and PV run.
    const int ntile = (a.Sk + KTS - 1) / KTS;
    if (wave < ntile) load(wave * KTS);
    for (int it = wave; it < ntile; it += NSPLIT) {
        const int kb = it * KTS;
        store_v();
        __builtin_amdgcn_wave_barrier();
        floatx16 s[1];
        s[0] = floatx16{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            s[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks], qf[ks], s[0], 0, 0, 0);
        // wave priority as in attn_kernel: the next tile's loads first, then the softmax / PV
        __builtin_amdgcn_s_setprio(2);
        if (it + NSPLIT < ntile) load(kb + NSPLIT * KTS);
        __builtin_amdgcn_s_setprio(1);
        // causal: query q0 + lrow sees keys up to itself
        const int kv = a.causal ? min(KTS, min(a.Sk, q0 + lrow + 1) - kb) : min(KTS, a.Sk - kb);
        softmax_pv<1, MTD, LSUM, kTRV>(s, kv, c, m_run, l_run, o, vt, VS, hl, lrow, lk, vlo);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_wave_barrier();
    }

    // merge: per wave (max, sum) per query and O^T partials [dim][query] in fp32
    const float l_tot = row_sum<MTD, LSUM>(o, l_run, lrow);
    __syncthreads();  // every wave is done with its V^T tile
    float* Ow = (float*)smem;                       // [NSPLIT][MTD*32][32]
    float* Mw = Ow + NSPLIT * MTD * 32 * 32;        // [NSPLIT][32]
    float* Lw = Mw + NSPLIT * 32;                   // [NSPLIT][32]
#pragma unroll
    for (int t = 0; t < MTD; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int dim = t * 32 + (e >> 2) * 8 + hl * 4 + (e & 3);
            Ow[(wave * MTD * 32 + dim) * 32 + lrow] = o[t][e];
        }
    if (hl == 0) {
        Mw[wave * 32 + lrow] = m_run;
        Lw[wave * 32 + lrow] = l_tot;
    }
    __syncthreads();
    // each thread produces 8 consecutive dims of one query
    const int nch = 32 * dch;
    for (int i = tid; i < nch; i += NTH) {
        const int q = i & 31, dc = i >> 5;
        if (q0 + q >= a.Sq) continue;
        float mmax = -INFINITY;
#pragma unroll
        for (int w = 0; w < NSPLIT; ++w) mmax = fmaxf(mmax, Mw[w * 32 + q]);
        float wt[NSPLIT], lsum = 0.f;
#pragma unroll
        for (int w = 0; w < NSPLIT; ++w) {
            wt[w] = fast_exp2(Mw[w * 32 + q] - mmax);  // an idle wave: -inf -> 0
            lsum += wt[w] * Lw[w * 32 + q];
        }
        const float inv = 1.0f / lsum;
        uint4 outv;
        f16* ov = (f16*)&outv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float acc = 0.f;
#pragma unroll
            for (int w = 0; w < NSPLIT; ++w) acc += wt[w] * Ow[(w * MTD * 32 + dc * 8 + e) * 32 + q];
            ov[e] = (f16)(acc * inv);
        }
        *(uint4*)(a.o + ((int64_t)b * a.Sq + q0 + q) * a.ldo + (int64_t)h * d + dc * 8) = outv;
    }
}

// ----------------------------------------------------------------- launch

// Blocks of one shared-tile variant resident on the whole chip at once (its occupancy
// per CU times the CUs), queried once per variant (the template arguments name it).
template <int KS, int MTD, bool LSUM, bool OFS, class Kern>
static int resident_blocks(Kern kern, int threads) {
    static int n = -1;
    if (n < 0) {
        int dev = 0, cus = 0, per = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kern, threads, 0) != hipSuccess)
            cus = per = 0;
        n = cus * per;
    }
    return n;
}

// How a launch runs: the shared-tile kernel (waves per block, 128-key tiles, the softmax
// reference in a spare dimension, keys split in two) or the key-split kernel (waves per
// 32-query group).
struct AttnPlan {
    bool shared;
    int nw, ns;
    bool kt128, ofs, spl;
    dim3 grid;
};

template <int KS, int MTD, bool LSUM>
static AttnPlan attn_plan(const AttnArgs& a) {
    AttnPlan p{};
    const int64_t bh = (int64_t)a.heads * a.B;
    const int64_t qwaves = ((a.Sq + 31) / 32) * bh;  // one wave per 32 queries
    // shared K/V tiles where there are enough query waves to fill the chip (the
    // key-split kernel re-reads K/V per wave): four query waves per block, eight for
    // heads of 56..128 when four would leave < 512 blocks (their larger K/V tiles are
    // then shared by more waves; measured per shape: d80 at 2304 tokens, B=2, 0.43 ms
    // with two waves, 0.375 with four, 0.353 with eight; d160 at 256 tokens, B=16, 0.221
    // with two, 0.158 with four).  Fewer query waves (e.g. 1024 queries x 16 heads), and
    // short key sequences (cross-attention over the 77 context tokens), go to the
    // key-split kernel: its extra waves, or not staging a few K/V tiles per block, win.
    if (qwaves >= 1024 && a.Sk > 128 && !a.causal) {
        p.shared = true;
        p.nw = (a.d > 48 && a.d <= 128 && ((a.Sq + 127) / 128) * bh < 512) ? 8 : 4;
        p.grid = dim3((a.Sq + p.nw * 32 - 1) / (p.nw * 32), a.heads, a.B);
        // 128-key tiles for heads <= 48 when every block is resident at once (two per CU):
        // d40 at 4096 tokens, B=2, 0.44 ms per forward against 0.46 with 64-key tiles;
        // on larger grids they lose (0.24 ms more at 9216 tokens, 0.31 ms at B=16)
        p.kt128 = KS == 3 && p.nw == 4 && (long)p.grid.x * bh <= 512;
        // the softmax reference rides in a spare head dimension when Q is pre-scaled
        p.ofs = a.q_log2 && a.d < KS * 16 && p.nw == 4;
        // Keys split in two when the blocks fill a round and a part of the next: the
        // half-length blocks then fill whole rounds.  A partial last round is modelled
        // at 3/4 of a full one's time, the merge at 1/20 (d40 at 9216 tokens, B=2: 1.5
        // rounds of 768 blocks; measured 1.75 round-times)
        if (p.nw == 4 && !p.kt128 && a.Sk > 64 && (long)p.grid.x * bh <= kAttnMaxPairs) {
            const long nblk = (long)p.grid.x * bh;
            const int slots = p.ofs ? resident_blocks<KS, MTD, LSUM, true>(attn_kernel<KS, MTD, 4, LSUM, 64, true, false, kTRV>, 256)
                                    : resident_blocks<KS, MTD, LSUM, false>(attn_kernel<KS, MTD, 4, LSUM, 64, false, false, kTRV>, 256);
            if (slots > 0) {
                auto rounds = [&](double r) { const double f = floor(r); return f + (r > f ? 0.75 : 0.0); };
                p.spl = rounds(2.0 * nblk / slots) * 0.5 + 0.05 < 0.9 * rounds((double)nblk / slots);
            }
        }
        return p;
    }
    // key split: enough waves to fill the chip, at most one per 32-key tile, and at
    // most 4 for wide heads (LDS for the fp32 merge)
    const int ntile = (a.Sk + KTS - 1) / KTS;
    int ns = (int)((2048 + qwaves - 1) / qwaves);
    if (ns > ntile) ns = ntile;
    const int nmax = MTD > 3 ? 4 : 8;
    p.ns = ns <= 1 ? 1 : ns <= 2 ? 2 : (ns <= 4 || nmax == 4) ? 4 : 8;
    p.grid = dim3((a.Sq + 31) / 32, a.heads, a.B);
    return p;
}

template <int KS, int MTD, bool LSUM>
static size_t ws_bytes(const AttnArgs& a) {
    const AttnPlan p = attn_plan<KS, MTD, LSUM>(a);
    if (!p.spl) return 0;
    const size_t pairs = (size_t)p.grid.x * p.grid.y * p.grid.z;
    return kAttnCounterFloats * 4 + pairs * 2 * 4 * (MTD * 16 + 2) * 64 * 4;  // attn_kernel's SPL slots
}

template <int KS, int MTD, bool LSUM>
static void launch_cfg(const AttnArgs& a0, hipStream_t s) {
    AttnArgs a = a0;
    const AttnPlan p = attn_plan<KS, MTD, LSUM>(a);
    const int64_t bh = (int64_t)a.heads * a.B;
    const double flops = 4.0 * bh * a.Sq * a.Sk * a.d;
    const double bytes = 2.0 * bh * a.d * (2.0 * a.Sq + 2.0 * a.Sk);
    char name[48];
    if (p.shared) {
        const bool spl = p.spl && a.ws;
        const bool trv = kTRV && !p.kt128;
        snprintf(name, sizeof name, "attn_kernel<%d,%d,%d,%d,%d,%d,%d,%d>", KS, MTD, p.nw, (int)LSUM, p.kt128 ? 128 : 64,
                 (int)p.ofs, (int)spl, (int)trv);
        constexpr int KTB = KS == 3 ? 128 : 64;
        dim3 grid = p.grid;
        if (spl) {
            a.kpart = ((a.Sk + 127) / 128) * 64;  // half the 64-key tiles (rounded up)
            grid.z *= 2;
        }
        launch_timed(name, flops, bytes, [&] {
            if (p.nw == 8) SDU_LAUNCH((attn_kernel<KS, MTD, 8, LSUM, 64, false, false, kTRV>), grid, dim3(512), 0, s, a);
            else if (KS == 3 && p.kt128 && p.ofs)
                SDU_LAUNCH((attn_kernel<KS, MTD, 4, LSUM, KTB, true>), grid, dim3(256), 0, s, a);
            else if (KS == 3 && p.kt128)
                SDU_LAUNCH((attn_kernel<KS, MTD, 4, LSUM, KTB>), grid, dim3(256), 0, s, a);
            else if (spl && p.ofs) SDU_LAUNCH((attn_kernel<KS, MTD, 4, LSUM, 64, true, true, kTRV>), grid, dim3(256), 0, s, a);
            else if (spl) SDU_LAUNCH((attn_kernel<KS, MTD, 4, LSUM, 64, false, true, kTRV>), grid, dim3(256), 0, s, a);
            else if (p.ofs) SDU_LAUNCH((attn_kernel<KS, MTD, 4, LSUM, 64, true, false, kTRV>), grid, dim3(256), 0, s, a);
            else SDU_LAUNCH((attn_kernel<KS, MTD, 4, LSUM, 64, false, false, kTRV>), grid, dim3(256), 0, s, a);
        });
        return;
    }
    const int ns = p.ns;
    snprintf(name, sizeof name, "attn_split_kernel<%d,%d,%d,%d>", KS, MTD, ns, (int)LSUM);
    const dim3 grid = p.grid;
    launch_timed(name, flops, bytes, [&] {
        if (ns == 1) SDU_LAUNCH((attn_split_kernel<KS, MTD, 1, LSUM>), grid, dim3(64), 0, s, a);
        else if (ns == 2) SDU_LAUNCH((attn_split_kernel<KS, MTD, 2, LSUM>), grid, dim3(128), 0, s, a);
        else if (ns == 4) SDU_LAUNCH((attn_split_kernel<KS, MTD, 4, LSUM>), grid, dim3(256), 0, s, a);
        else SDU_LAUNCH((attn_split_kernel<KS, MTD, (MTD > 3 ? 4 : 8), LSUM>), grid,
                                dim3(64 * (MTD > 3 ? 4 : 8)), 0, s, a);
    });
}

template <int KS, int MTD>
static void launch_d(const AttnArgs& a, hipStream_t s) {
    if (a.d < MTD * 32) launch_cfg<KS, MTD, true>(a, s);
    else launch_cfg<KS, MTD, false>(a, s);
}

template <int KS, int MTD>
static size_t ws_d(const AttnArgs& a) {
    return a.d < MTD * 32 ? ws_bytes<KS, MTD, true>(a) : ws_bytes<KS, MTD, false>(a);
}

size_t attention_workspace_bytes(const AttnArgs& a) {
    if (a.d <= 0 || a.d > 160 || (a.d & 7) || a.Sq <= 0 || a.Sk <= 0) return 0;
    const int d = a.d;
    if (d <= 32) return ws_d<2, 1>(a);
    if (d <= 48) return ws_d<3, 2>(a);
    if (d <= 64) return ws_d<4, 2>(a);
    if (d <= 80) return ws_d<5, 3>(a);
    if (d <= 96) return ws_d<6, 3>(a);
    if (d <= 128) return ws_d<8, 4>(a);
    return ws_d<10, 5>(a);
}

hipError_t attention_launch(const AttnArgs& a, hipStream_t s) {
    if (a.d <= 0 || a.d > 160 || (a.d & 7) || a.Sq <= 0 || a.Sk <= 0 || !(a.scale > 0.f) ||
        (a.causal && a.Sq != a.Sk))
        return hipErrorInvalidValue;
    const int d = a.d;
    if (d <= 32) launch_d<2, 1>(a, s);
    else if (d <= 48) launch_d<3, 2>(a, s);
    else if (d <= 64) launch_d<4, 2>(a, s);
    else if (d <= 80) launch_d<5, 3>(a, s);
    else if (d <= 96) launch_d<6, 3>(a, s);
    else if (d <= 128) launch_d<8, 4>(a, s);
    else launch_d<10, 5>(a, s);
    return hipGetLastError();
}

}  // namespace sdu
