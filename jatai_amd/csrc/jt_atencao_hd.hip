// Causal ALiBi attention for heads of width HD = 64 (and any multiple of 16): the declared generalization of the
// spec's head-width-4 attention (ops.py:186-258), which it reduces to at HD = 4 (the oracle checks that reduction):
//   alignment: values of head h aligned to the largest block exponent the head spans over the T tokens;
//   score:     u_ij = rnd(q_i . k_j, -(eq + ek - log2(HD)/2 + 8)) - (i - j) << incl,  incl = 8 - 8h/H;
//   dS:        shrunk to DSB = 12 - max(0, log2 T - 7) bits (keeps |gq|, |gk| < 2^30 at T = 256).
//
// Aligned values satisfy |a| <= 127 << 4 = 2032, so they are stored as int16 and every dot product over the
// head width runs on v_dot2_i32_i16 (two exact 16-bit products per op, int32 accumulation: |q.k| < 64 * 2032^2
// < 2^28). Each row (query or key) is owned by a quad of 4 lanes holding HD/4 consecutive dimensions; a quad
// reduces a dot product with two intra-quad shuffles, so the 4 lanes then agree on the score, and each lane
// accumulates outputs for its own dimensions (no cross-lane reduction of output vectors).
//
// Forward: one workgroup of 256 threads per (sequence, head, block of 64 query rows); keys [0, 64 qb + 64)
// staged in LDS. Backward: the spec needs two maxima over a whole (sequence, head) -- the causal max |gP| that
// sets gP's 15-bit shrink and the max |dS| that sets dS's shrink -- so it runs as four launches over the same
// (sequence, head, 64-row block) grid: (1) partial maxima of |gP| (or the LIMITE variant's bound terms),
// (2) s_i = rnd(sum_j P gP', 8) and partial maxima of |dS| (or its bound terms), (3) gq for the block's query
// rows and gk, gv for its key rows, (4) the exponent columns. The partial maxima and s_i live, between
// launches, in the op's own output: the exponent area of the gv columns, which launch (4) writes last.
#include "jt_comum.h"

typedef short s2_t __attribute__((ext_vector_type(2)));

namespace hd {
constexpr int QB = 64;                 // query (or key) rows per workgroup
constexpr int NT = 4 * QB;             // 256 threads: one quad per row
}

__device__ __forceinline__ int dot2(int a, int b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2_t, a), __builtin_bit_cast(s2_t, b), c, false);
}
__device__ __forceinline__ int quad_soma(int v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    return v;
}
__device__ __forceinline__ int lo16(int w) { return (int)(short)(w & 0xffff); }
__device__ __forceinline__ int hi16(int w) { return w >> 16; }

// workgroup maximum (blockDim.x a multiple of 64, red sized blockDim.x / 64)
__device__ __forceinline__ int wg_max(int v, int* red) {
    v = g_max<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = SEM_TOPO;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) r = max(r, red[i]);
    return r;
}

// Largest block exponent head slice [col0, col0 + HD) spans over the T tokens of sequence b0 / T.
template <int HD>
__device__ __forceinline__ int emx_cabeca(const int8_t* E, int ld, int col0, int blk, int b0, int T, int* red) {
    constexpr int DL = HD / 4;
    const int r = threadIdx.x & 3, nbl = ld / blk, cb = (col0 + DL * r) / blk;
    int m = SEM_TOPO;
    for (int t = threadIdx.x >> 2; t < T; t += blockDim.x >> 2) m = max(m, (int)E[(size_t)(b0 + t) * nbl + cb]);
    return wg_max(m, red);
}

// This lane's DL aligned values of token row `tok` (absolute row index), packed as int16 pairs.
template <int HD>
__device__ __forceinline__ void alinha_lane(const int8_t* m, const int8_t* E, int ld, int col0, int blk, int tok, int emx, int GA,
                                            int (&w)[HD / 8]) {
    constexpr int DL = HD / 4;
    const int r = threadIdx.x & 3, c = col0 + DL * r;
    const int s = emx - (int)E[(size_t)tok * (ld / blk) + c / blk];
    int v[DL];
    le_i8(m + (size_t)tok * ld + c, v);
#pragma unroll
    for (int k = 0; k < DL / 2; k++) {
        const int a0 = rnd_d(v[2 * k] << GA, s), a1 = rnd_d(v[2 * k + 1] << GA, s);
        w[k] = (a0 & 0xffff) | (a1 << 16);
    }
}

// ---------------------------------------------------------------------------------------------- forward
template <int HD>
__global__ void __launch_bounds__(hd::NT) k_atencao_hd(const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, int* __restrict__ Oacc,
                                                       int16_t* __restrict__ Oe, uint8_t* __restrict__ P, int T, int H, int D, int blk, int GA,
                                                       int kid) {
    using namespace hd;
    constexpr int DL = HD / 4, W = HD / 8;                          // values per lane, int16-pair words per lane
    extern __shared__ __align__(16) int sm_hd[];
    int* ka = sm_hd;                                                // [keys][HD/2] words
    int* va = ka + (size_t)T * (HD / 2);
    __shared__ int red[NT / 64];
    const int nqb = T / QB, bh = blockIdx.x / nqb, qb = blockIdx.x % nqb, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, quad = threadIdx.x >> 2, r = threadIdx.x & 3;
    const int i = qb * QB + quad, row = b0 + i, tk = qb * QB + QB;
    const int emq = emx_cabeca<HD>(qE, ld, h * HD, blk, b0, T, red);
    const int emk = emx_cabeca<HD>(qE, ld, D + h * HD, blk, b0, T, red);
    const int emv = emx_cabeca<HD>(qE, ld, 2 * D + h * HD, blk, b0, T, red);
    for (int t = quad; t < tk; t += QB) {
        int w[W];
        alinha_lane<HD>(qm, qE, ld, D + h * HD, blk, b0 + t, emk, GA, w);
#pragma unroll
        for (int k = 0; k < W; k++) ka[t * (HD / 2) + r * W + k] = w[k];
        alinha_lane<HD>(qm, qE, ld, 2 * D + h * HD, blk, b0 + t, emv, GA, w);
#pragma unroll
        for (int k = 0; k < W; k++) va[t * (HD / 2) + r * W + k] = w[k];
    }
    int q[W];
    alinha_lane<HD>(qm, qE, ld, h * HD, blk, row, emq, GA, q);
    __syncthreads();
    const int eq = emq - GA, ek = emk - GA, ev = emv - GA;
    const int su = -(eq + ek - ilog2_c(HD) / 2 + 8), incl = 8 - (8 * h) / H;
    const long long idx = (long long)row * D + h * HD;
    auto u_ij = [&](int j) {
        const int* kr = ka + j * (HD / 2) + r * W;
        int s = 0;
#pragma unroll
        for (int k = 0; k < W; k++) s = dot2(q[k], kr[k], s);
        s = quad_soma(s);
        return rnd(s, su, kid, idx) - ((i - j) << incl);
    };
    int mx = U_MIN;
    for (int j = 0; j <= i; j++) mx = max(mx, u_ij(j));
    int soma = 0;
    for (int j = 0; j <= i; j++) soma += exp_dif(mx, u_ij(j)) >> 3;
    if (soma <= 0) { if (r == 0) reporta(E_DIV, kid, idx, soma, mx); soma = 1; }
    const int inv = (1 << 28) / soma;
    int o[DL];
#pragma unroll
    for (int k = 0; k < DL; k++) o[k] = 0;
    uint8_t* Pb = P + (size_t)bh * T * T;
    for (int j = 0; j <= i; j++) {
        const int p = min(((exp_dif(mx, u_ij(j)) >> 3) * inv + (1 << 19)) >> 20, 255);
        if (r == 0) Pb[(size_t)j * T + i] = (uint8_t)p;
        const int* vr = va + j * (HD / 2) + r * W;
#pragma unroll
        for (int k = 0; k < W; k++) { o[2 * k] += p * lo16(vr[k]); o[2 * k + 1] += p * hi16(vr[k]); }
    }
    if (r == 0)
        for (int j = i + 1; j < T; j++) Pb[(size_t)j * T + i] = 0;
    const size_t x = (size_t)row * D + h * HD + DL * r;
    int16_t eo[DL];
#pragma unroll
    for (int k = 0; k < DL; k++) {
        if (o[k] >= LIM || o[k] <= -LIM) reporta(E_ACUM, kid, x + k, o[k], -3);
        eo[k] = (int16_t)(ev - 8);
    }
#pragma unroll
    for (int k = 0; k < DL; k += 4) *reinterpret_cast<int4*>(Oacc + x + k) = make_int4(o[k], o[k + 1], o[k + 2], o[k + 3]);
    grava_i16(Oe + x, eo);
}

// ---------------------------------------------------------------------------------------------- backward
// Scratch slots (int32) inside Ge's gv columns of sequence b, head h: row b*T + t, byte offset
// ((b*T + t) * 3D + 2D + h*HD) * 2; slot 0 of row t holds s_t, slots 1.. of row qb hold block qb's partials.
__device__ __forceinline__ int* slot_hd(int16_t* Ge, int b0, int t, int D, int h, int HDv) {
    return reinterpret_cast<int*>(Ge + (size_t)(b0 + t) * 3 * D + 2 * D + h * HDv);
}

struct CabecaHd {                       // per (sequence, head) constants shared by the backward launches
    int ego, eq, ek, ev;
};

template <int HD>
__device__ __forceinline__ CabecaHd cabeca_hd(const int8_t* gE, const int8_t* qE, int D, int h, int blk, int b0, int T, int GA, int* red) {
    CabecaHd c;
    c.ego = emx_cabeca<HD>(gE, D, h * HD, blk, b0, T, red) - GA;
    c.eq = emx_cabeca<HD>(qE, 3 * D, h * HD, blk, b0, T, red) - GA;
    c.ek = emx_cabeca<HD>(qE, 3 * D, D + h * HD, blk, b0, T, red) - GA;
    c.ev = emx_cabeca<HD>(qE, 3 * D, 2 * D + h * HD, blk, b0, T, red) - GA;
    return c;
}

// (1) partial maxima: exact |gP| over the block's causal pairs, or the bound terms max||dO_i||_inf and
//     max||v_j||_1 over the block's tokens (ops.py:231-235)
template <int HD, int LIMITE>
__global__ void __launch_bounds__(hd::NT) k_atb_max1(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE,
                                                     const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, int16_t* __restrict__ Ge,
                                                     int T, int H, int D, int blk, int GA) {
    using namespace hd;
    constexpr int W = HD / 8;
    extern __shared__ __align__(16) int sm_hd[];
    int* va = sm_hd;
    __shared__ int red[NT / 64];
    const int nqb = T / QB, bh = blockIdx.x / nqb, qb = blockIdx.x % nqb, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, quad = threadIdx.x >> 2, r = threadIdx.x & 3, i = qb * QB + quad;
    const int emg = emx_cabeca<HD>(goE, D, h * HD, blk, b0, T, red);
    const int emv = emx_cabeca<HD>(qE, ld, 2 * D + h * HD, blk, b0, T, red);
    int g[W];
    alinha_lane<HD>(gom, goE, D, h * HD, blk, b0 + i, emg, GA, g);
    int* sl = slot_hd(Ge, b0, qb, D, h, HD);
    if constexpr (LIMITE) {
        int v[W];
        alinha_lane<HD>(qm, qE, ld, 2 * D + h * HD, blk, b0 + i, emv, GA, v);
        int a1 = 0, a2 = 0;
#pragma unroll
        for (int k = 0; k < W; k++) {
            a1 = max(a1, max(abs(lo16(g[k])), abs(hi16(g[k]))));
            a2 += abs(lo16(v[k])) + abs(hi16(v[k]));
        }
        a2 = quad_soma(a2);
        a1 = wg_max(a1, red);
        a2 = wg_max(a2, red);
        if (threadIdx.x == 0) { sl[1] = a1; sl[2] = a2; }
        return;
    }
    for (int t = quad; t < qb * QB + QB; t += QB) {
        int w[W];
        alinha_lane<HD>(qm, qE, ld, 2 * D + h * HD, blk, b0 + t, emv, GA, w);
#pragma unroll
        for (int k = 0; k < W; k++) va[t * (HD / 2) + r * W + k] = w[k];
    }
    __syncthreads();
    int mg = 0;
    for (int j = 0; j <= i; j++) {
        const int* vr = va + j * (HD / 2) + r * W;
        int s = 0;
#pragma unroll
        for (int k = 0; k < W; k++) s = dot2(g[k], vr[k], s);
        mg = max(mg, abs(quad_soma(s)));
    }
    mg = wg_max(mg, red);
    if (threadIdx.x == 0) sl[1] = mg;
}

// shift of gP from the partials of launch (1)
template <int LIMITE>
__device__ __forceinline__ int sh_gp(int16_t* Ge, int b0, int D, int h, int HDv, int nqb) {
    int a = 0, c = 0;
    for (int q = 0; q < nqb; q++) {
        const int* s = slot_hd(Ge, b0, q, D, h, HDv);
        a = max(a, s[1]);
        if (LIMITE) c = max(c, s[2]);
    }
    return max(bitlen(LIMITE ? a * c : a) - 15, 0);
}

// (2) s_i = rnd(sum_j P_ij rnd(gP_ij, sh), 8) for the block's rows, and partial maxima for dS's shrink
template <int HD, int LIMITE>
__global__ void __launch_bounds__(hd::NT) k_atb_slin(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE,
                                                     const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, const uint8_t* __restrict__ P,
                                                     int16_t* __restrict__ Ge, int T, int H, int D, int blk, int GA, int kid) {
    using namespace hd;
    constexpr int W = HD / 8;
    extern __shared__ __align__(16) int sm_hd[];
    int* va = sm_hd;
    __shared__ int red[NT / 64];
    const int nqb = T / QB, bh = blockIdx.x / nqb, qb = blockIdx.x % nqb, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, quad = threadIdx.x >> 2, r = threadIdx.x & 3, i = qb * QB + quad;
    const int emg = emx_cabeca<HD>(goE, D, h * HD, blk, b0, T, red);
    const int emv = emx_cabeca<HD>(qE, ld, 2 * D + h * HD, blk, b0, T, red);
    for (int t = quad; t < qb * QB + QB; t += QB) {
        int w[W];
        alinha_lane<HD>(qm, qE, ld, 2 * D + h * HD, blk, b0 + t, emv, GA, w);
#pragma unroll
        for (int k = 0; k < W; k++) va[t * (HD / 2) + r * W + k] = w[k];
    }
    int g[W];
    alinha_lane<HD>(gom, goE, D, h * HD, blk, b0 + i, emg, GA, g);
    const int sh = sh_gp<LIMITE>(Ge, b0, D, h, HD, nqb);
    __syncthreads();                                                // partials read by every thread before any write below
    const uint8_t* Pb = P + (size_t)bh * T * T;
    auto gp = [&](int j) {
        const int* vr = va + j * (HD / 2) + r * W;
        int s = 0;
#pragma unroll
        for (int k = 0; k < W; k++) s = dot2(g[k], vr[k], s);
        return rnd_d(quad_soma(s), sh);
    };
    int s = 0, pm = 0, gm = 0;
    for (int j = 0; j <= i; j++) {
        const int p = Pb[(size_t)j * T + i], x = gp(j);
        s += p * x;
        if (LIMITE) { pm = max(pm, p); gm = max(gm, abs(x)); }
    }
    if ((s >= LIM || s <= -LIM) && r == 0) reporta(E_ACUM, kid, (long long)(b0 + i) * ld + h * HD, s, -4);
    const int sl = rnd_d(s, 8);
    int* slq = slot_hd(Ge, b0, qb, D, h, HD);
    if constexpr (LIMITE) {
        pm = wg_max(pm, red);
        gm = wg_max(gm, red);
        const int smx = wg_max(abs(sl), red);
        if (threadIdx.x == 0) { slq[3] = pm; slq[4] = gm; slq[5] = smx; }
    } else {
        int md = 0;
        for (int j = 0; j <= i; j++) md = max(md, abs((int)Pb[(size_t)j * T + i] * (gp(j) - sl)));
        md = wg_max(md, red);
        if (threadIdx.x == 0) slq[3] = md;
    }
    if (r == 0) slot_hd(Ge, b0, i, D, h, HD)[0] = sl;
}

// shift of dS from the partials of launch (2)
template <int LIMITE>
__device__ __forceinline__ int sh_ds(int16_t* Ge, int b0, int D, int h, int HDv, int nqb, int dsb) {
    int a = 0, c = 0, d = 0;
    for (int q = 0; q < nqb; q++) {
        const int* s = slot_hd(Ge, b0, q, D, h, HDv);
        a = max(a, s[3]);
        if (LIMITE) { c = max(c, s[4]); d = max(d, s[5]); }
    }
    return max(bitlen(LIMITE ? a * (c + d) : a) - dsb, 0);
}

// (3) gq_i = sum_{j <= i} dS_ij k_j for the block's query rows; gk_j = sum_{i >= j} dS_ij q_i and
//     gv_j = sum_{i >= j} P_ij dO_i for the block's key rows. Writes Gacc only.
template <int HD, int LIMITE>
__global__ void __launch_bounds__(hd::NT) k_atb_grad(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE,
                                                     const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, const uint8_t* __restrict__ P,
                                                     int* __restrict__ Gacc, int16_t* __restrict__ Ge, int T, int H, int D, int blk, int GA,
                                                     int dsb, int kid) {
    using namespace hd;
    constexpr int DL = HD / 4, W = HD / 8;
    extern __shared__ __align__(16) int sm_hd[];
    const int nqb = T / QB, bh = blockIdx.x / nqb, qb = blockIdx.x % nqb, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, quad = threadIdx.x >> 2, r = threadIdx.x & 3;
    const int nk = qb * QB + QB, q0 = qb * QB, nq = T - q0;         // keys [0, nk); queries [q0, T)
    int* ka = sm_hd;                                                // [nk][HD/2]
    int* va = ka + (size_t)nk * (HD / 2);
    int* goa = va + (size_t)nk * (HD / 2);                          // [nq][HD/2], row t - q0
    int* qa = goa + (size_t)nq * (HD / 2);
    int* slin = qa + (size_t)nq * (HD / 2);                         // [nq]
    __shared__ int red[NT / 64];
    const CabecaHd c = cabeca_hd<HD>(goE, qE, D, h, blk, b0, T, GA, red);
    const int emg = c.ego + GA, emq = c.eq + GA, emk = c.ek + GA, emv = c.ev + GA;
    for (int t = quad; t < nk; t += QB) {
        int w[W];
        alinha_lane<HD>(qm, qE, ld, D + h * HD, blk, b0 + t, emk, GA, w);
#pragma unroll
        for (int k = 0; k < W; k++) ka[t * (HD / 2) + r * W + k] = w[k];
        alinha_lane<HD>(qm, qE, ld, 2 * D + h * HD, blk, b0 + t, emv, GA, w);
#pragma unroll
        for (int k = 0; k < W; k++) va[t * (HD / 2) + r * W + k] = w[k];
    }
    for (int t = quad; t < nq; t += QB) {
        int w[W];
        alinha_lane<HD>(gom, goE, D, h * HD, blk, b0 + q0 + t, emg, GA, w);
#pragma unroll
        for (int k = 0; k < W; k++) goa[t * (HD / 2) + r * W + k] = w[k];
        alinha_lane<HD>(qm, qE, ld, h * HD, blk, b0 + q0 + t, emq, GA, w);
#pragma unroll
        for (int k = 0; k < W; k++) qa[t * (HD / 2) + r * W + k] = w[k];
    }
    for (int t = threadIdx.x; t < nq; t += NT) slin[t] = slot_hd(Ge, b0, q0 + t, D, h, HD)[0];
    const int sh = sh_gp<LIMITE>(Ge, b0, D, h, HD, nqb);
    const int sh2 = sh_ds<LIMITE>(Ge, b0, D, h, HD, nqb, dsb);
    __syncthreads();
    const uint8_t* Pb = P + (size_t)bh * T * T;
    // rows: query i = q0 + quad
    {
        const int i = q0 + quad, il = quad;
        const int* gi = goa + il * (HD / 2) + r * W;
        const int sl = slin[il];
        int gq[DL];
#pragma unroll
        for (int k = 0; k < DL; k++) gq[k] = 0;
        for (int j = 0; j <= i; j++) {
            const int* vr = va + j * (HD / 2) + r * W;
            int s = 0;
#pragma unroll
            for (int k = 0; k < W; k++) s = dot2(gi[k], vr[k], s);
            const int ds = rnd_d((int)Pb[(size_t)j * T + i] * (rnd_d(quad_soma(s), sh) - sl), sh2);
            const int* kr = ka + j * (HD / 2) + r * W;
#pragma unroll
            for (int k = 0; k < W; k++) { gq[2 * k] += ds * lo16(kr[k]); gq[2 * k + 1] += ds * hi16(kr[k]); }
        }
        const size_t o = (size_t)(b0 + i) * ld + h * HD + DL * r;
#pragma unroll
        for (int k = 0; k < DL; k++)
            if (gq[k] >= LIM || gq[k] <= -LIM) reporta(E_ACUM, kid, o + k, gq[k], -5);
#pragma unroll
        for (int k = 0; k < DL; k += 4) *reinterpret_cast<int4*>(Gacc + o + k) = make_int4(gq[k], gq[k + 1], gq[k + 2], gq[k + 3]);
    }
    // columns: key j = q0 + quad (the block's own rows)
    {
        const int j = q0 + quad;
        const int* vj = va + j * (HD / 2) + r * W;
        int vreg[W];
#pragma unroll
        for (int k = 0; k < W; k++) vreg[k] = vj[k];
        int gk[DL], gv[DL];
#pragma unroll
        for (int k = 0; k < DL; k++) { gk[k] = 0; gv[k] = 0; }
        const uint8_t* Pr = Pb + (size_t)j * T;
        for (int i = j; i < T; i++) {
            const int il = i - q0;
            const int* gi = goa + il * (HD / 2) + r * W;
            int s = 0;
#pragma unroll
            for (int k = 0; k < W; k++) s = dot2(gi[k], vreg[k], s);
            const int p = Pr[i];
            const int ds = rnd_d(p * (rnd_d(quad_soma(s), sh) - slin[il]), sh2);
            const int* qi = qa + il * (HD / 2) + r * W;
#pragma unroll
            for (int k = 0; k < W; k++) {
                gk[2 * k] += ds * lo16(qi[k]); gk[2 * k + 1] += ds * hi16(qi[k]);
                gv[2 * k] += p * lo16(gi[k]); gv[2 * k + 1] += p * hi16(gi[k]);
            }
        }
        const size_t o = (size_t)(b0 + j) * ld + h * HD + DL * r;
#pragma unroll
        for (int k = 0; k < DL; k++) {
            if (gk[k] >= LIM || gk[k] <= -LIM) reporta(E_ACUM, kid, o + D + k, gk[k], -5);
            if (gv[k] >= LIM || gv[k] <= -LIM) reporta(E_ACUM, kid, o + 2 * D + k, gv[k], -5);
        }
#pragma unroll
        for (int k = 0; k < DL; k += 4) {
            *reinterpret_cast<int4*>(Gacc + o + D + k) = make_int4(gk[k], gk[k + 1], gk[k + 2], gk[k + 3]);
            *reinterpret_cast<int4*>(Gacc + o + 2 * D + k) = make_int4(gv[k], gv[k + 1], gv[k + 2], gv[k + 3]);
        }
    }
}

// (4) exponent columns of head h: eds + ek (gq), eds + eq (gk), ego - 8 (gv). One workgroup per
//     (sequence, head) reads the partials first and only then overwrites the scratch area.
template <int HD, int LIMITE>
__global__ void __launch_bounds__(hd::NT) k_atb_exp(const int8_t* __restrict__ goE, const int8_t* __restrict__ qE, int16_t* __restrict__ Ge,
                                                    int T, int H, int D, int blk, int GA, int dsb) {
    using namespace hd;
    constexpr int DL = HD / 4;
    __shared__ int red[NT / 64];
    const int bh = blockIdx.x, b = bh / H, h = bh % H, b0 = b * T, nqb = T / QB, r = threadIdx.x & 3;
    const CabecaHd c = cabeca_hd<HD>(goE, qE, D, h, blk, b0, T, GA, red);
    const int sh = sh_gp<LIMITE>(Ge, b0, D, h, HD, nqb);
    const int sh2 = sh_ds<LIMITE>(Ge, b0, D, h, HD, nqb, dsb);
    const int eds = c.ego + c.ev + sh - 9 + sh2;
    __syncthreads();
    int16_t a[DL], bq[DL], cv[DL];
#pragma unroll
    for (int k = 0; k < DL; k++) { a[k] = (int16_t)(eds + c.ek); bq[k] = (int16_t)(eds + c.eq); cv[k] = (int16_t)(c.ego - 8); }
    for (int t = threadIdx.x >> 2; t < T; t += NT / 4) {
        const size_t o = (size_t)(b0 + t) * 3 * D + h * HD + DL * r;
        grava_i16(Ge + o, a);
        grava_i16(Ge + o + D, bq);
        grava_i16(Ge + o + 2 * D, cv);
    }
}
