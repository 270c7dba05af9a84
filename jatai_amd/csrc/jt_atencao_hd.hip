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
// The scalar products are 24-bit ones (mul24): P <= 255, ex <= 4095 and 2^28 / sum ex <= 2^16 (the row maximum
// alone adds 4095 to the sum), |gP' - s| < 2^17 (|gP'| <= 2^15, a row of P sums to at most 256 + T / 2).
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
    const int passo = blockDim.x >> 2;
    int t = threadIdx.x >> 2;
    for (; t + 3 * passo < T; t += 4 * passo) {                      // four independent loads per round
        const int8_t* e = E + (size_t)(b0 + t) * nbl + cb;
        m = max(max(m, (int)e[0]), max((int)e[(size_t)passo * nbl], max((int)e[(size_t)2 * passo * nbl], (int)e[(size_t)3 * passo * nbl])));
    }
    for (; t < T; t += passo) m = max(m, (int)E[(size_t)(b0 + t) * nbl + cb]);
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
        const int a0 = rnd_d(shl(v[2 * k], GA), s), a1 = rnd_d(shl(v[2 * k + 1], GA), s);
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
        const int p = min((mul24(exp_dif(mx, u_ij(j)) >> 3, inv) + (1 << 19)) >> 20, 255);
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
            const int ds = rnd_d(mul24(p, rnd_d(quad_soma(s), sh) - slin[il]), sh2);
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

// ---------------------------------------------------------------------------------------------- forward on MFMA (HD = 64)
// Same arithmetic as k_atencao_hd, computed with matrix cores. An aligned value a = rnd(m << GA, s) is exactly
// m8 << L with m8 int8 and L >= 0 per (token, 32-dimension half): (m, GA - s) if s <= GA, else (rnd(m, s - GA), 0)
// (the reference's packing, jatai_cuda.cu:789-818). So q_i . k_j = sum over the two halves c of
// (m8q_i . m8k_j)_c << (Lq_ic + Lk_jc): one i8 MFMA 16x16x32 per half and tile, shifted and added exactly in
// int32 (|(.)_c| < 2^19, shift <= 8). The scores of a wave's 16 query rows stay in registers (16 per key tile),
// so max, sum and P take one pass each over them. PV runs as an f16 MFMA 16x16x32: P <= 255 and |v| <= 2032
// are exact in f16, products exact in fp32, and every partial sum is bounded by sum_j P_ij * 2032 < 2^20 (the
// P of a row sum to at most 256 + T/2), so the fp32 accumulation is exact and converts back to the same int.
// Workgroup = 4 waves = 64 query rows of one (sequence, head); wave w owns rows 16 w .. 16 w + 15.
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void m8_L(int m, int s, int GA, int& m8, int& L) {
    if (s <= GA) { m8 = m; L = GA - s; }
    else { m8 = rnd_d(m, s - GA); L = 0; }
}

template <int TMAX>
__global__ void __launch_bounds__(256) k_atencao_mf(const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, int* __restrict__ Oacc,
                                                    int16_t* __restrict__ Oe, uint8_t* __restrict__ P, int T, int H, int D, int blk, int GA,
                                                    int kid) {
    constexpr int HD = 64, NTT = TMAX / 16;
    extern __shared__ __align__(16) char sm_mf[];
    const int nqb = T / 64, bh = blockIdx.x / nqb, qb = blockIdx.x % nqb, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, Tk = qb * 64 + 64, nbl = ld / blk;
    int8_t* km = reinterpret_cast<int8_t*>(sm_mf);                  // [Tk][64] m8 of k
    int8_t* kL = km + (size_t)Tk * 64;                              // [Tk][2] L of k per half
    _Float16* vt = reinterpret_cast<_Float16*>(kL + (((size_t)Tk * 2 + 15) & ~(size_t)15));   // [64][Tk] aligned v, transposed
    _Float16* ps = vt + (size_t)64 * Tk;                            // [4][16][Tk] P of each wave
    __shared__ int red[4];
    __shared__ int qL[64][2];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int emq = emx_cabeca<HD>(qE, ld, h * HD, blk, b0, T, red);
    const int emk = emx_cabeca<HD>(qE, ld, D + h * HD, blk, b0, T, red);
    const int emv = emx_cabeca<HD>(qE, ld, 2 * D + h * HD, blk, b0, T, red);
    // k and v of tokens [0, Tk): thread (t, c4) handles dimensions 16 c4 .. 16 c4 + 15 of token t
    for (int t = tid >> 2; t < Tk; t += 64) {
        const int c4 = tid & 3, half = c4 >> 1;
        const size_t base = (size_t)(b0 + t) * ld;
        int v[16];
        le_i8(qm + base + D + h * HD + 16 * c4, v);
        const int sk = emk - (int)qE[(size_t)(b0 + t) * nbl + (D + h * HD + 16 * c4) / blk];
        int8_t m8[16];
        int L = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) { int a; m8_L(v[k], sk, GA, a, L); m8[k] = (int8_t)a; }
        grava_i8(km + (size_t)t * 64 + 16 * c4, m8);
        if ((c4 & 1) == 0) kL[t * 2 + half] = (int8_t)L;
        le_i8(qm + base + 2 * D + h * HD + 16 * c4, v);
        const int sv = emv - (int)qE[(size_t)(b0 + t) * nbl + (2 * D + h * HD + 16 * c4) / blk];
#pragma unroll
        for (int k = 0; k < 16; k++) vt[(size_t)(16 * c4 + k) * Tk + t] = (_Float16)rnd_d(shl(v[k], GA), sv);
    }
    // q fragments: A row lr = query row 16 w + lr, dimensions 32 c + 8 lg .. + 7 of half c
    const int ia = qb * 64 + 16 * w + lr;
    long qa[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int col = h * HD + 32 * c + 8 * lg;
        int v[8];
        le_i8(qm + (size_t)(b0 + ia) * ld + col, v);
        const int s = emq - (int)qE[(size_t)(b0 + ia) * nbl + col / blk];
        long pk = 0;
        int L = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) { int a; m8_L(v[k], s, GA, a, L); pk |= (long)(uint8_t)a << (8 * k); }
        qa[c] = pk;
        if (lg == 0) qL[16 * w + lr][c] = L;
    }
    __syncthreads();
    const int eq = emq - GA, ek = emk - GA, ev = emv - GA;
    const int su = -(eq + ek - 3 + 8), incl = 8 - (8 * h) / H;     // log2(64) / 2 = 3
    const int i0 = qb * 64 + 16 * w + 4 * lg;                        // this lane's 4 score rows: i0 .. i0 + 3
    int lq[4][2];
#pragma unroll
    for (int v = 0; v < 4; v++) { lq[v][0] = qL[16 * w + 4 * lg + v][0]; lq[v][1] = qL[16 * w + 4 * lg + v][1]; }
    const int ntk = qb * 4 + w + 1;                                  // key tiles [0, 16 ntk) reach the wave's last row
    const long long idx = (long long)(b0 + i0) * D + h * HD;
    int uu[NTT][4], mx[4] = {U_MIN, U_MIN, U_MIN, U_MIN};
#pragma unroll
    for (int t = 0; t < NTT; t++) {
        if (t >= ntk) continue;                                      // guarded, not break: uu stays in registers
        const int j = 16 * t + lr;
        const long kb0 = *reinterpret_cast<const long*>(km + (size_t)j * 64 + 8 * lg);
        const long kb1 = *reinterpret_cast<const long*>(km + (size_t)j * 64 + 32 + 8 * lg);
        const int lk0 = kL[j * 2], lk1 = kL[j * 2 + 1];
        const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa[0], kb0, v4i{0, 0, 0, 0}, 0, 0, 0);
        const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa[1], kb1, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int i = i0 + v;
            const int s = shl(p0[v], lq[v][0] + lk0) + shl(p1[v], lq[v][1] + lk1);
            const int r = su >= 0 ? rnd_d(s, su) : rnd(s, su, kid, idx);
            const int u = j <= i ? r - ((i - j) << incl) : U_MIN;
            uu[t][v] = u;
            mx[v] = max(mx[v], u);
        }
    }
#pragma unroll
    for (int v = 0; v < 4; v++) mx[v] = g_max<16>(mx[v]);
    int soma[4] = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NTT; t++) {
        if (t >= ntk) continue;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int ex = uu[t][v] == U_MIN ? 0 : exp_dif(mx[v], uu[t][v]) >> 3;
            uu[t][v] = ex;
            soma[v] += ex;
        }
    }
    int inv[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        int s = g_sum<16>(soma[v]);
        if (s <= 0) { if (lr == 0) reporta(E_DIV, kid, idx + (long long)v * D, s, mx[v]); s = 1; }
        inv[v] = (1 << 28) / s;
    }
    uint8_t* Pb = P + (size_t)bh * T * T;
    _Float16* pw = ps + (size_t)w * 16 * Tk;
#pragma unroll
    for (int t = 0; t < NTT; t++) {
        if (t >= ntk) continue;
        const int j = 16 * t + lr;
        unsigned pk = 0;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int p = min((mul24(uu[t][v], inv[v]) + (1 << 19)) >> 20, 255);
            pk |= (unsigned)p << (8 * v);
            pw[(size_t)(4 * lg + v) * Tk + j] = (_Float16)p;
        }
        *reinterpret_cast<unsigned*>(Pb + (size_t)j * T + i0) = pk;
    }
    for (int t = ntk; t < T / 16; t++) *reinterpret_cast<unsigned*>(Pb + (size_t)(16 * t + lr) * T + i0) = 0u;
    if (ntk & 1)
#pragma unroll
        for (int v = 0; v < 4; v++) pw[(size_t)(4 * lg + v) * Tk + 16 * ntk + lr] = (_Float16)0;
    __syncthreads();
    // O = P V on f16 MFMA: A = P rows lr, keys 32 ch + 8 lg ..; B = v^T dims 16 dt + lr, same keys
    f4_t o[4] = {};
    const int nch = (ntk + 1) / 2;
    for (int ch = 0; ch < nch; ch++) {
        const h8_t a = *reinterpret_cast<const h8_t*>(pw + (size_t)lr * Tk + 32 * ch + 8 * lg);
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            const h8_t bv = *reinterpret_cast<const h8_t*>(vt + (size_t)(16 * dt + lr) * Tk + 32 * ch + 8 * lg);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bv, o[dt], 0, 0, 0);
        }
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const size_t x = (size_t)(b0 + i0 + v) * D + h * HD + 16 * dt + lr;
            const int ov = (int)o[dt][v];
            if (ov >= LIM || ov <= -LIM) reporta(E_ACUM, kid, x, ov, -3);
            Oacc[x] = ov;
            Oe[x] = (int16_t)(ev - 8);
        }
}

// ---------------------------------------------------------------------------------------------- backward on MFMA (HD = 64)
// Same arithmetic as the dot2 backward above, with matrix cores:
//   gP (or gP^T) tiles: i8 MFMA per 32-dimension half on the m8 << L packing, shifted and added in int32;
//   gq = dS K and gk = dS^T Q: f16 MFMA with dS (|dS| < 2^12) split as a 256 + b 16 + c, a in [-16, 15],
//     b, c in [0, 15], so each piece times |k| <= 2032 and summed over <= 256 terms stays below 2^24: exact
//     in fp32; the three exact sums are recombined in int32;
//   gv = P^T dO: f16 MFMA with P split as 16 ph + pl (pieces <= 15; a column of P is not bounded by 256).
// Launch B3r computes gq for a block's query rows, B3c gk and gv for a block's key rows (one writer per output).
typedef short s8_t __attribute__((ext_vector_type(8)));

// m8 bytes of dimensions 32 c + 8 g .. + 7 of head slice col0 for token row tok, and L of that half
__device__ __forceinline__ long m8L_frag(const int8_t* m, const int8_t* E, int ld, int col0, int blk, int tok, int emx, int GA, int c, int g,
                                         int& L) {
    const int col = col0 + 32 * c + 8 * g;
    int v[8];
    le_i8(m + (size_t)tok * ld + col, v);
    const int s = emx - (int)E[(size_t)tok * (ld / blk) + col / blk];
    long pk = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) { int a; m8_L(v[k], s, GA, a, L); pk |= (long)(uint8_t)a << (8 * k); }
    return pk;
}

// Stage rows [t0, t0 + n) of a head slice as m8 [n][64] + L [n][2] (threads 4 per row)
__device__ __forceinline__ void estagia_m8(const int8_t* m, const int8_t* E, int ld, int col0, int blk, int b0, int t0, int n, int emx, int GA,
                                           int8_t* dm, int8_t* dL) {
    for (int t = threadIdx.x >> 2; t < n; t += blockDim.x >> 2) {
        const int c4 = threadIdx.x & 3;
        int v[16];
        le_i8(m + (size_t)(b0 + t0 + t) * ld + col0 + 16 * c4, v);
        const int s = emx - (int)E[(size_t)(b0 + t0 + t) * (ld / blk) + (col0 + 16 * c4) / blk];
        int8_t m8[16];
        int L = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) { int a; m8_L(v[k], s, GA, a, L); m8[k] = (int8_t)a; }
        grava_i8(dm + (size_t)t * 64 + 16 * c4, m8);
        if ((c4 & 1) == 0) dL[t * 2 + (c4 >> 1)] = (int8_t)L;
    }
}

// Stage rows [t0, t0 + n) of a head slice as aligned f16, transposed: dt[d][t] (stride n)
__device__ __forceinline__ void estagia_f16t(const int8_t* m, const int8_t* E, int ld, int col0, int blk, int b0, int t0, int n, int emx, int GA,
                                             _Float16* dt) {
    for (int t = threadIdx.x >> 2; t < n; t += blockDim.x >> 2) {
        const int c4 = threadIdx.x & 3;
        int v[16];
        le_i8(m + (size_t)(b0 + t0 + t) * ld + col0 + 16 * c4, v);
        const int s = emx - (int)E[(size_t)(b0 + t0 + t) * (ld / blk) + (col0 + 16 * c4) / blk];
#pragma unroll
        for (int k = 0; k < 16; k++) dt[(size_t)(16 * c4 + k) * n + t] = (_Float16)rnd_d(shl(v[k], GA), s);
    }
}

// 16 x 16 tile of X Y^T over the 64 head dimensions from m8 fragments: lane (lr, lg) gets rows 4 lg + v, column lr
__device__ __forceinline__ void tile_xyt(long xa0, long xa1, long yb0, long yb1, const int (&lx)[4][2], int ly0, int ly1, int (&out)[4]) {
    const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa0, yb0, v4i{0, 0, 0, 0}, 0, 0, 0);
    const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa1, yb1, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 4; v++) out[v] = shl(p0[v], lx[v][0] + ly0) + shl(p1[v], lx[v][1] + ly1);
}

// The exact fp32 piece sums (integers below 2^23) back to an integer: a 256 + b 16 + c and a 16 + b. (int) of an
// integral float is one conversion; (long long) of a float would be a ten-instruction sequence per value. The
// recombined value is a sum of at most 256 terms |dS| |k| <= 4096 * 2032 (or P |dO| <= 255 * 2032), below 2^31,
// so the 32-bit arithmetic (modular: unsigned) gives it exactly.
__device__ __forceinline__ int junta3(float a, float b, float c) {
    return (int)((unsigned)(int)a * 256u + (unsigned)(int)b * 16u + (unsigned)(int)c);
}
__device__ __forceinline__ int junta2(float a, float b) { return (int)((unsigned)(int)a * 16u + (unsigned)(int)b); }

// f16 pieces of 8 int16 dS values: dS = a 256 + b 16 + c
__device__ __forceinline__ void pedacos_ds(const s8_t& d, h8_t& a, h8_t& b, h8_t& c) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int x = d[k];
        a[k] = (_Float16)(x >> 8);
        b[k] = (_Float16)((x >> 4) & 15);
        c[k] = (_Float16)(x & 15);
    }
}

// B1/B2 (rows of query block qb; PASSO 1: max |gP|; PASSO 2: s_i and the dS maxima). LIMITE runs only PASSO 2.
template <int TMAX, int PASSO, int LIMITE>
__global__ void __launch_bounds__(256) k_atb_mf_linhas(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE,
                                                       const int8_t* __restrict__ qm, const int8_t* __restrict__ qE,
                                                       const uint8_t* __restrict__ P, int16_t* __restrict__ Ge, int T, int H, int D, int blk,
                                                       int GA, int kid) {
    constexpr int HD = 64, NTT = TMAX / 16;
    extern __shared__ __align__(16) char sm_mf[];
    const int nqb = T / 64, bh = blockIdx.x / nqb, qb = blockIdx.x % nqb, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, Tk = qb * 64 + 64;
    int8_t* vm = reinterpret_cast<int8_t*>(sm_mf);                  // [Tk][64]
    int8_t* vL = vm + (size_t)Tk * 64;                              // [Tk][2]
    __shared__ int red[4];
    __shared__ int gL[64][2];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int emg = emx_cabeca<HD>(goE, D, h * HD, blk, b0, T, red);
    const int emv = emx_cabeca<HD>(qE, ld, 2 * D + h * HD, blk, b0, T, red);
    estagia_m8(qm, qE, ld, 2 * D + h * HD, blk, b0, 0, Tk, emv, GA, vm, vL);
    const int ia = qb * 64 + 16 * w + lr;
    long ga[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        int L;
        ga[c] = m8L_frag(gom, goE, D, h * HD, blk, b0 + ia, emg, GA, c, lg, L);
        if (lg == 0) gL[16 * w + lr][c] = L;
    }
    int sh = 0;
    if (PASSO == 2) sh = sh_gp<LIMITE>(Ge, b0, D, h, HD, nqb);
    __syncthreads();
    int lx[4][2];
#pragma unroll
    for (int v = 0; v < 4; v++) { lx[v][0] = gL[16 * w + 4 * lg + v][0]; lx[v][1] = gL[16 * w + 4 * lg + v][1]; }
    const int i0 = qb * 64 + 16 * w + 4 * lg, ntk = qb * 4 + w + 1;
    const uint8_t* Pb = P + (size_t)bh * T * T;
    int g[NTT][4];
    int mg = 0, s[4] = {0, 0, 0, 0}, pm = 0, gm = 0;
    unsigned pr[NTT];
#pragma unroll
    for (int t = 0; t < NTT; t++) {
        if (t >= ntk) continue;
        const int j = 16 * t + lr;
        int o[4];
        tile_xyt(ga[0], ga[1], *reinterpret_cast<const long*>(vm + (size_t)j * 64 + 8 * lg),
                 *reinterpret_cast<const long*>(vm + (size_t)j * 64 + 32 + 8 * lg), lx, vL[j * 2], vL[j * 2 + 1], o);
        if (PASSO == 1) {
#pragma unroll
            for (int v = 0; v < 4; v++) if (j <= i0 + v) mg = max(mg, abs(o[v]));
        } else {
            pr[t] = *reinterpret_cast<const unsigned*>(Pb + (size_t)j * T + i0);      // P_ij of rows i0 .. i0 + 3 (0 above the diagonal)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int x = j <= i0 + v ? rnd_d(o[v], sh) : 0;
                const int p = (pr[t] >> (8 * v)) & 255;
                g[t][v] = x;
                s[v] += p * x;
                if (LIMITE) { pm = max(pm, p); gm = max(gm, abs(x)); }
            }
        }
    }
    int* slq = slot_hd(Ge, b0, qb, D, h, HD);
    if (PASSO == 1) {
        mg = wg_max(mg, red);
        if (tid == 0) slq[1] = mg;
        return;
    }
    int sl[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int tot = g_sum<16>(s[v]);
        if ((tot >= LIM || tot <= -LIM) && lr == 0) reporta(E_ACUM, kid, (long long)(b0 + i0 + v) * ld + h * HD, tot, -4);
        sl[v] = rnd_d(tot, 8);
        if (lr == 0) slot_hd(Ge, b0, i0 + v, D, h, HD)[0] = sl[v];
    }
    if (LIMITE) {
        pm = wg_max(pm, red);
        gm = wg_max(gm, red);
        const int smx = wg_max(max(max(abs(sl[0]), abs(sl[1])), max(abs(sl[2]), abs(sl[3]))), red);
        if (tid == 0) { slq[3] = pm; slq[4] = gm; slq[5] = smx; }
    } else {
        int md = 0;
#pragma unroll
        for (int t = 0; t < NTT; t++) {
            if (t >= ntk) continue;
#pragma unroll
            for (int v = 0; v < 4; v++) md = max(md, abs(mul24((int)((pr[t] >> (8 * v)) & 255), g[t][v] - sl[v])));
        }
        md = wg_max(md, red);
        if (tid == 0) slq[3] = md;
    }
}

// B3r: gq_i = sum_{j <= i} dS_ij k_j for the query rows of block qb
template <int TMAX, int LIMITE>
__global__ void __launch_bounds__(256) k_atb_mf_gq(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE, const int8_t* __restrict__ qm,
                                                   const int8_t* __restrict__ qE, const uint8_t* __restrict__ P, int* __restrict__ Gacc,
                                                   int16_t* __restrict__ Ge, int T, int H, int D, int blk, int GA, int dsb, int kid) {
    constexpr int HD = 64, NTT = TMAX / 16;
    extern __shared__ __align__(16) char sm_mf[];
    const int nqb = T / 64, bh = blockIdx.x / nqb, qb = blockIdx.x % nqb, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, Tk = qb * 64 + 64;
    int8_t* vm = reinterpret_cast<int8_t*>(sm_mf);                  // [Tk][64]
    int8_t* vL = vm + (size_t)Tk * 64;                              // [Tk][2]
    _Float16* kt = reinterpret_cast<_Float16*>(vL + (((size_t)Tk * 2 + 15) & ~(size_t)15));   // [64][Tk]
    short* dsw = reinterpret_cast<short*>(kt + (size_t)64 * Tk);    // [4][16][Tk]
    __shared__ int red[4];
    __shared__ int gL[64][2];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const CabecaHd cb = cabeca_hd<HD>(goE, qE, D, h, blk, b0, T, GA, red);
    estagia_m8(qm, qE, ld, 2 * D + h * HD, blk, b0, 0, Tk, cb.ev + GA, GA, vm, vL);
    estagia_f16t(qm, qE, ld, D + h * HD, blk, b0, 0, Tk, cb.ek + GA, GA, kt);
    const int ia = qb * 64 + 16 * w + lr;
    long ga[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        int L;
        ga[c] = m8L_frag(gom, goE, D, h * HD, blk, b0 + ia, cb.ego + GA, GA, c, lg, L);
        if (lg == 0) gL[16 * w + lr][c] = L;
    }
    const int sh = sh_gp<LIMITE>(Ge, b0, D, h, HD, nqb), sh2 = sh_ds<LIMITE>(Ge, b0, D, h, HD, nqb, dsb);
    const int i0 = qb * 64 + 16 * w + 4 * lg, ntk = qb * 4 + w + 1;
    int sl[4];
#pragma unroll
    for (int v = 0; v < 4; v++) sl[v] = slot_hd(Ge, b0, i0 + v, D, h, HD)[0];
    __syncthreads();
    int lx[4][2];
#pragma unroll
    for (int v = 0; v < 4; v++) { lx[v][0] = gL[16 * w + 4 * lg + v][0]; lx[v][1] = gL[16 * w + 4 * lg + v][1]; }
    const uint8_t* Pb = P + (size_t)bh * T * T;
    short* dw = dsw + (size_t)w * 16 * Tk;
#pragma unroll
    for (int t = 0; t < NTT; t++) {
        if (t >= ntk) continue;
        const int j = 16 * t + lr;
        int o[4];
        tile_xyt(ga[0], ga[1], *reinterpret_cast<const long*>(vm + (size_t)j * 64 + 8 * lg),
                 *reinterpret_cast<const long*>(vm + (size_t)j * 64 + 32 + 8 * lg), lx, vL[j * 2], vL[j * 2 + 1], o);
        const unsigned pr = *reinterpret_cast<const unsigned*>(Pb + (size_t)j * T + i0);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int p = (pr >> (8 * v)) & 255;
            const int ds = j <= i0 + v ? rnd_d(mul24(p, rnd_d(o[v], sh) - sl[v]), sh2) : 0;
            dw[(size_t)(4 * lg + v) * Tk + j] = (short)ds;
        }
    }
    if (ntk & 1)
#pragma unroll
        for (int v = 0; v < 4; v++) dw[(size_t)(4 * lg + v) * Tk + 16 * ntk + lr] = 0;
    __syncthreads();
    f4_t acc[4][3] = {};
    const int nch = (ntk + 1) / 2;
    for (int ch = 0; ch < nch; ch++) {
        h8_t pa, pb, pc;
        pedacos_ds(*reinterpret_cast<const s8_t*>(dw + (size_t)lr * Tk + 32 * ch + 8 * lg), pa, pb, pc);
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            const h8_t kv = *reinterpret_cast<const h8_t*>(kt + (size_t)(16 * dt + lr) * Tk + 32 * ch + 8 * lg);
            acc[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, kv, acc[dt][0], 0, 0, 0);
            acc[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pb, kv, acc[dt][1], 0, 0, 0);
            acc[dt][2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pc, kv, acc[dt][2], 0, 0, 0);
        }
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const long long gq = junta3(acc[dt][0][v], acc[dt][1][v], acc[dt][2][v]);
            const size_t o = (size_t)(b0 + i0 + v) * ld + h * HD + 16 * dt + lr;
            if (gq >= LIM || gq <= -LIM) reporta(E_ACUM, kid, o, gq, -5);
            Gacc[o] = (int)gq;
        }
}

// B3c: gk_j = sum_{i >= j} dS_ij q_i and gv_j = sum_{i >= j} P_ij dO_i for the key rows of block kb
template <int TMAX, int LIMITE>
__global__ void __launch_bounds__(256) k_atb_mf_gkv(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE, const int8_t* __restrict__ qm,
                                                    const int8_t* __restrict__ qE, const uint8_t* __restrict__ P, int* __restrict__ Gacc,
                                                    int16_t* __restrict__ Ge, int T, int H, int D, int blk, int GA, int dsb, int kid) {
    constexpr int HD = 64, NTT = TMAX / 16;
    extern __shared__ __align__(16) char sm_mf[];
    const int nqb = T / 64, bh = blockIdx.x / nqb, kb = blockIdx.x % nqb, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, q0 = kb * 64, nq = T - q0;     // queries [q0, T)
    int8_t* gm8 = reinterpret_cast<int8_t*>(sm_mf);                 // dO m8 [nq][64]
    int8_t* gL8 = gm8 + (size_t)nq * 64;                            // [nq][2]
    _Float16* qt = reinterpret_cast<_Float16*>(gL8 + (((size_t)nq * 2 + 15) & ~(size_t)15));  // [64][nq]
    _Float16* gt = qt + (size_t)64 * nq;                            // dO aligned [64][nq]
    short* dsw = reinterpret_cast<short*>(gt + (size_t)64 * nq);    // [4][16][nq] dS^T
    uint8_t* pw = reinterpret_cast<uint8_t*>(dsw + (size_t)4 * 16 * nq);   // [4][16][nq] P^T
    int* slv = reinterpret_cast<int*>(pw + (size_t)4 * 16 * nq);    // [nq]
    __shared__ int red[4];
    __shared__ int vLs[64][2];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const CabecaHd cb = cabeca_hd<HD>(goE, qE, D, h, blk, b0, T, GA, red);
    estagia_m8(gom, goE, D, h * HD, blk, b0, q0, nq, cb.ego + GA, GA, gm8, gL8);
    estagia_f16t(qm, qE, ld, h * HD, blk, b0, q0, nq, cb.eq + GA, GA, qt);
    estagia_f16t(gom, goE, D, h * HD, blk, b0, q0, nq, cb.ego + GA, GA, gt);
    for (int t = tid; t < nq; t += 256) slv[t] = slot_hd(Ge, b0, q0 + t, D, h, HD)[0];
    // v fragments of this wave's 16 keys j0 + lr as the A operand (rows = keys)
    const int j0 = q0 + 16 * w, ja = j0 + lr;
    long va[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        int L;
        va[c] = m8L_frag(qm, qE, ld, 2 * D + h * HD, blk, b0 + ja, cb.ev + GA, GA, c, lg, L);
        if (lg == 0) vLs[16 * w + lr][c] = L;
    }
    const int sh = sh_gp<LIMITE>(Ge, b0, D, h, HD, nqb), sh2 = sh_ds<LIMITE>(Ge, b0, D, h, HD, nqb, dsb);
    __syncthreads();
    int lx[4][2];
#pragma unroll
    for (int v = 0; v < 4; v++) { lx[v][0] = vLs[16 * w + 4 * lg + v][0]; lx[v][1] = vLs[16 * w + 4 * lg + v][1]; }
    const int jr = j0 + 4 * lg;                                      // this lane's 4 keys: jr .. jr + 3
    const uint8_t* Pb = P + (size_t)bh * T * T;
    short* dw = dsw + (size_t)w * 16 * nq;
    uint8_t* pww = pw + (size_t)w * 16 * nq;
    const int t0 = w, nt = nq / 16;                                  // query tiles [t0, nt) (relative to q0) reach keys >= j0
    for (int t = 0; t < t0; t++)                                     // tiles before the diagonal: zero
#pragma unroll
        for (int v = 0; v < 4; v++) { dw[(size_t)(4 * lg + v) * nq + 16 * t + lr] = 0; pww[(size_t)(4 * lg + v) * nq + 16 * t + lr] = 0; }
#pragma unroll
    for (int t = 0; t < NTT; t++) {
        if (t < t0 || t >= nt) continue;
        const int il = 16 * t + lr, i = q0 + il;                     // this lane's query (column)
        int o[4];
        tile_xyt(va[0], va[1], *reinterpret_cast<const long*>(gm8 + (size_t)il * 64 + 8 * lg),
                 *reinterpret_cast<const long*>(gm8 + (size_t)il * 64 + 32 + 8 * lg), lx, gL8[il * 2], gL8[il * 2 + 1], o);
        const int sl = slv[il];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int j = jr + v;
            const int p = i >= j ? (int)Pb[(size_t)j * T + i] : 0;
            const int ds = i >= j ? rnd_d(mul24(p, rnd_d(o[v], sh) - sl), sh2) : 0;
            dw[(size_t)(4 * lg + v) * nq + il] = (short)ds;
            pww[(size_t)(4 * lg + v) * nq + il] = (uint8_t)p;
        }
    }
    __syncthreads();
    f4_t ak[4][3] = {}, av[4][2] = {};
    for (int ch = (16 * t0) / 32; ch < nq / 32; ch++) {
        h8_t pa, pb, pc, ph, pl;
        pedacos_ds(*reinterpret_cast<const s8_t*>(dw + (size_t)lr * nq + 32 * ch + 8 * lg), pa, pb, pc);
        const uint8_t* pp = pww + (size_t)lr * nq + 32 * ch + 8 * lg;
#pragma unroll
        for (int k = 0; k < 8; k++) { ph[k] = (_Float16)(pp[k] >> 4); pl[k] = (_Float16)(pp[k] & 15); }
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            const h8_t qv = *reinterpret_cast<const h8_t*>(qt + (size_t)(16 * dt + lr) * nq + 32 * ch + 8 * lg);
            const h8_t gv = *reinterpret_cast<const h8_t*>(gt + (size_t)(16 * dt + lr) * nq + 32 * ch + 8 * lg);
            ak[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, qv, ak[dt][0], 0, 0, 0);
            ak[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pb, qv, ak[dt][1], 0, 0, 0);
            ak[dt][2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pc, qv, ak[dt][2], 0, 0, 0);
            av[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, gv, av[dt][0], 0, 0, 0);
            av[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, gv, av[dt][1], 0, 0, 0);
        }
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const long long gk = junta3(ak[dt][0][v], ak[dt][1][v], ak[dt][2][v]);
            const long long gvv = junta2(av[dt][0][v], av[dt][1][v]);
            const size_t o = (size_t)(b0 + jr + v) * ld + h * HD + 16 * dt + lr;
            if (gk >= LIM || gk <= -LIM) reporta(E_ACUM, kid, o + D, gk, -5);
            if (gvv >= LIM || gvv <= -LIM) reporta(E_ACUM, kid, o + 2 * D, gvv, -5);
            Gacc[o + D] = (int)gk;
            Gacc[o + 2 * D] = (int)gvv;
        }
}
