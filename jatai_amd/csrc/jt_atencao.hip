// Causal ALiBi attention at head width 4 (the spec's shape, ops.py:186-258): one workgroup per
// (sequence, head), one thread per query row i. T is a multiple of 32 up to 256; the workgroup has T rounded up
// to whole waves of 64 threads, and the threads past T take part in the reductions with neutral values only.
//
// Forward: q, k, v of the head aligned to the head's largest exponent over the sequence with GA guard bits
// (a = rnd(m << GA, emx - e)); u_ij = rnd(q_i . k_j, -(eq + ek - 1 + 8)) - (i - j) << incl with
// incl = 8 - h // 8 (ops.py:208; H <= 64); ex = exp_int(max - u) >> 3; P = min((ex * (2^28 / sum ex) + 2^19) >> 20, 255) as uint8,
// stored transposed [j][i]; o_i = sum_j P_ij v_j (raw, exponent ev - 8).
// Backward: gP = dO . v^T shrunk to 15 bits by its causal maximum (or an upper bound in the LIMITE variant),
// s_i = rnd(sum_j P gP, 8), dS = P (gP - s) shrunk to DSB bits, then gq = dS k, gk = dS^T q, gv = P^T dO
// as raw outputs [M, 3D].
#include "jt_comum.h"

__device__ __forceinline__ int bloco_max(int v, int* red) {
    v = g_max<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = SEM_TOPO;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) r = max(r, red[i]);
    return r;
}

// aligned values of this thread's token for one head slice of 4 columns (jatai_cuda.cu:789-818 restated);
// a thread past the sequence (t >= T) loads nothing and holds zeros
__device__ __forceinline__ void alinha4(const int8_t* m, const int8_t* E, int ld, int col, int blk, int b0, int T, int GA, int* red,
                                        int (*al)[4], int& eo) {
    const int t = threadIdx.x;
    const bool ativo = t < T;
    const int e = ativo ? (int)E[(size_t)(b0 + t) * (ld / blk) + col / blk] : SEM_TOPO;
    const int emx = bloco_max(e, red);
    const int w = ativo ? *reinterpret_cast<const int*>(m + (size_t)(b0 + t) * ld + col) : 0;
#pragma unroll
    for (int d = 0; d < 4; d++) al[t][d] = ativo ? rnd_d(((w << (24 - 8 * d)) >> 24) << GA, emx - e) : 0;
    eo = emx - GA;
}

template <int TMAX>
__global__ void __launch_bounds__(TMAX) k_atencao4(const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, int* __restrict__ Oacc,
                                                   int16_t* __restrict__ Oe, uint8_t* __restrict__ P, int T, int H, int D, int blk, int GA,
                                                   int kid) {
    __shared__ int qa[TMAX][4], ka[TMAX][4], va[TMAX][4];
    __shared__ int red[TMAX / 64];
    const int b = blockIdx.x / H, h = blockIdx.x % H, ld = 3 * D, b0 = b * T;
    int eq, ek, ev;
    alinha4(qm, qE, ld, h * 4, blk, b0, T, GA, red, qa, eq);
    alinha4(qm, qE, ld, D + h * 4, blk, b0, T, GA, red, ka, ek);
    alinha4(qm, qE, ld, 2 * D + h * 4, blk, b0, T, GA, red, va, ev);
    __syncthreads();
    const int su = -(eq + ek - 1 + 8), incl = 8 - h / 8;
    const int i = threadIdx.x, row = b0 + i;
    if (i >= T) return;                                             // no barrier follows
    const int q0 = qa[i][0], q1 = qa[i][1], q2 = qa[i][2], q3 = qa[i][3];
    const long long idx = (long long)row * D + h * 4;
    auto sc = [&](int j) {
        const int s = q0 * ka[j][0] + q1 * ka[j][1] + q2 * ka[j][2] + q3 * ka[j][3];
        return rnd(s, su, kid, idx) - ((i - j) << incl);
    };
    int mx = U_MIN;
    for (int j = 0; j <= i; j++) mx = max(mx, sc(j));
    int soma = 0;
    for (int j = 0; j <= i; j++) soma += exp_dif(mx, sc(j)) >> 3;
    if (soma <= 0) { reporta(E_DIV, kid, idx, soma, mx); soma = 1; }
    const int inv = (1 << 28) / soma;
    int o[4] = {0, 0, 0, 0};
    uint8_t* Pb = P + (size_t)blockIdx.x * T * T;
    for (int j = 0; j < T; j++) {
        int p = 0;
        if (j <= i) {
            const int ex = exp_dif(mx, sc(j)) >> 3;
            p = min((ex * inv + (1 << 19)) >> 20, 255);
#pragma unroll
            for (int d = 0; d < 4; d++) o[d] += p * va[j][d];
        }
        Pb[(size_t)j * T + i] = (uint8_t)p;
    }
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const size_t x = (size_t)row * D + h * 4 + d;
        if (o[d] >= LIM || o[d] <= -LIM) reporta(E_ACUM, kid, x, o[d], -3);
        Oacc[x] = o[d];
        Oe[x] = (int16_t)(ev - 8);
    }
}

template <int TMAX, int LIMITE>
__global__ void __launch_bounds__(TMAX) k_atencao4_back(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE,
                                                        const int8_t* __restrict__ qm, const int8_t* __restrict__ qE,
                                                        const uint8_t* __restrict__ P, int* __restrict__ Gacc, int16_t* __restrict__ Ge,
                                                        int T, int H, int D, int blk, int GA, int DSB, int kid) {
    __shared__ int goa[TMAX][4], qa[TMAX][4], ka[TMAX][4], va[TMAX][4], slin[TMAX];
    __shared__ int red[TMAX / 64];
    const int b = blockIdx.x / H, h = blockIdx.x % H, ld = 3 * D, b0 = b * T;
    const uint8_t* Pb = P + (size_t)blockIdx.x * T * T;
    int eq, ek, ev, ego;
    alinha4(gom, goE, D, h * 4, blk, b0, T, GA, red, goa, ego);
    alinha4(qm, qE, ld, h * 4, blk, b0, T, GA, red, qa, eq);
    alinha4(qm, qE, ld, D + h * 4, blk, b0, T, GA, red, ka, ek);
    alinha4(qm, qE, ld, 2 * D + h * 4, blk, b0, T, GA, red, va, ev);
    __syncthreads();
    // threads past the sequence stay for the barriers of the reductions: their row loops are empty (ie = -1),
    // their aligned values zero, and they write nothing
    const int i = threadIdx.x, ie = i < T ? i : -1;
    const int g0 = goa[i][0], g1 = goa[i][1], g2 = goa[i][2], g3 = goa[i][3];
    auto gp_ij = [&](int j) { return g0 * va[j][0] + g1 * va[j][1] + g2 * va[j][2] + g3 * va[j][3]; };
    // shift of gP: exact causal maximum, or max_i ||dO_i||_inf * max_j ||v_j||_1
    int mg = 0;
    if constexpr (LIMITE) {
        const int b1 = max(max(abs(g0), abs(g1)), max(abs(g2), abs(g3)));
        const int b2 = abs(va[i][0]) + abs(va[i][1]) + abs(va[i][2]) + abs(va[i][3]);
        mg = bloco_max(b1, red) * bloco_max(b2, red);
    } else {
        for (int j = 0; j <= ie; j++) mg = max(mg, abs(gp_ij(j)));
        mg = bloco_max(mg, red);
    }
    const int sh = max(bitlen(mg) - 15, 0), egp = ego + ev + sh;
    // s_i = rnd(sum_j P_ij gP'_ij, 8)
    int s = 0, pm = 0, gm = 0;
    for (int j = 0; j <= ie; j++) {
        const int p = Pb[(size_t)j * T + i], gp = rnd_d(gp_ij(j), sh);
        s += p * gp;
        if constexpr (LIMITE) { pm = max(pm, p); gm = max(gm, abs(gp)); }
    }
    if (s >= LIM || s <= -LIM) reporta(E_ACUM, kid, (long long)(b0 + i) * ld + h * 4, s, -4);
    const int sl = rnd_d(s, 8);
    slin[i] = sl;
    // shift of dS: exact maximum of |P (gP' - s)|, or max P * (max |gP'| + max |s|)
    int md = 0;
    if constexpr (LIMITE) {
        const int pmb = bloco_max(pm, red), gmb = bloco_max(gm, red), smb = bloco_max(abs(sl), red);
        md = pmb * (gmb + smb);
    } else {
        for (int j = 0; j <= ie; j++) md = max(md, abs((int)Pb[(size_t)j * T + i] * (rnd_d(gp_ij(j), sh) - sl)));
        md = bloco_max(md, red);                                   // also publishes slin
    }
    const int sh2 = max(bitlen(md) - DSB, 0), eds = egp - 9 + sh2;
    // rows: gq_i = sum_j dS_ij k_j
    {
        int gq[4] = {0, 0, 0, 0};
        for (int j = 0; j <= ie; j++) {
            const int ds = rnd_d((int)Pb[(size_t)j * T + i] * (rnd_d(gp_ij(j), sh) - sl), sh2);
#pragma unroll
            for (int d = 0; d < 4; d++) gq[d] += ds * ka[j][d];
        }
        if (ie < 0) return;                                         // no barrier follows
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const size_t o = (size_t)(b0 + i) * ld + h * 4 + d;
            if (gq[d] >= LIM || gq[d] <= -LIM) reporta(E_ACUM, kid, o, gq[d], -5);
            Gacc[o] = gq[d];
            Ge[o] = (int16_t)(eds + ek);
        }
    }
    // columns: gk_j = sum_{i >= j} dS_ij q_i, gv_j = sum_{i >= j} P_ij dO_i (row j of the stored P is contiguous)
    {
        const int jj = threadIdx.x;
        const int v0 = va[jj][0], v1 = va[jj][1], v2 = va[jj][2], v3 = va[jj][3];
        const uint8_t* Pr = Pb + (size_t)jj * T;
        int gk[4] = {0, 0, 0, 0}, gv[4] = {0, 0, 0, 0};
        for (int ii = jj; ii < T; ii++) {
            const int p = Pr[ii];
            const int gp = goa[ii][0] * v0 + goa[ii][1] * v1 + goa[ii][2] * v2 + goa[ii][3] * v3;
            const int ds = rnd_d(p * (rnd_d(gp, sh) - slin[ii]), sh2);
#pragma unroll
            for (int d = 0; d < 4; d++) { gk[d] += ds * qa[ii][d]; gv[d] += p * goa[ii][d]; }
        }
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const size_t o = (size_t)(b0 + jj) * ld + h * 4 + d;
            if (gk[d] >= LIM || gk[d] <= -LIM) reporta(E_ACUM, kid, o + D, gk[d], -5);
            if (gv[d] >= LIM || gv[d] <= -LIM) reporta(E_ACUM, kid, o + 2 * D, gv[d], -5);
            Gacc[o + D] = gk[d];
            Ge[o + D] = (int16_t)(eds + eq);
            Gacc[o + 2 * D] = gv[d];
            Ge[o + 2 * D] = (int16_t)(ego - 8);
        }
    }
}
