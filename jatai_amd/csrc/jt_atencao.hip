// Causal ALiBi attention at head width 4 (the spec's shape, ops.py:186-258): one workgroup per
// (sequence, head), one or two query rows per thread. T is a multiple of 32 up to 256; the workgroup has T / NR
// threads rounded up to whole waves of 64, and the threads without a row take part in the reductions with
// neutral values only.
//
// Forward: q, k, v of the head aligned to the head's largest exponent over the sequence with GA guard bits
// (a = rnd(m << GA, emx - e)); u_ij = rnd(q_i . k_j, -(eq + ek - 1 + 8)) - (i - j) << incl with
// incl = 8 - h // 8 (ops.py:208; H <= 64); ex = exp_int(max - u) >> 3; P = min((ex * (2^28 / sum ex) + 2^19) >> 20, 255) as uint8,
// stored transposed [j][i]; o_i = sum_j P_ij v_j (raw, exponent ev - 8).
// Backward: gP = dO . v^T shrunk to 15 bits by its causal maximum (or an upper bound in the LIMITE variant),
// s_i = rnd(sum_j P gP, 8), dS = P (gP - s) shrunk to DSB bits, then gq = dS k, gk = dS^T q, gv = P^T dO
// as raw outputs [M, 3D].
// Every product is a 24-bit one (mul24): aligned values |a| <= 128 << GA <= 2048 (GA <= 4), P <= 255, ex <= 4095,
// 2^28 / sum ex <= 2^16 (the row maximum alone adds 4095 to the sum), |gP'| <= 2^15, |gP' - s| < 2^17 (a row of P
// sums to at most 256 + T / 2), |dS| <= 2^12.
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

// Rows per thread (jt_atencao_linhas, jatai_cuda.cu:1091): with NR = 1 thread t owns query row t; with NR = 2 it
// owns rows t and T - 1 - t (t < T / 2), a short and a long causal row, so the threads' work is even. The backward
// assigns its columns (keys) the same way. -1: no row (a thread past the sequence).
template <int NR>
__device__ __forceinline__ int linha_de(int t, int k, int T) {
    if constexpr (NR == 1) return t < T ? t : -1;
    else return t < T / 2 ? (k == 0 ? t : T - 1 - t) : -1;
}

// aligned values of the thread's tokens for one head slice of 4 columns (jatai_cuda.cu:789-818 restated):
// al[t][d] = rnd(m << GA, emx - e) with emx the head's largest exponent over the sequence; eo = emx - GA
template <int NR>
__device__ __forceinline__ void alinha4(const int8_t* m, const int8_t* E, int ld, int col, int blk, int b0, int T, int GA, int* red,
                                        int (*al)[4], int& eo) {
    int e[NR], w[NR], tk[NR], emx = SEM_TOPO;
#pragma unroll
    for (int k = 0; k < NR; k++) {
        tk[k] = linha_de<NR>(threadIdx.x, k, T);
        e[k] = tk[k] >= 0 ? (int)E[(size_t)(b0 + tk[k]) * (ld / blk) + col / blk] : SEM_TOPO;
        w[k] = tk[k] >= 0 ? *reinterpret_cast<const int*>(m + (size_t)(b0 + tk[k]) * ld + col) : 0;
        emx = max(emx, e[k]);
    }
    emx = bloco_max(emx, red);
#pragma unroll
    for (int k = 0; k < NR; k++)
        if (tk[k] >= 0) {
#pragma unroll
            for (int d = 0; d < 4; d++) al[tk[k]][d] = rnd_d(((w[k] << (24 - 8 * d)) >> 24) << GA, emx - e[k]);
        }
    eo = emx - GA;
}

template <int TMAX, int NR>
__global__ void __launch_bounds__(TMAX) k_atencao4(const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, int* __restrict__ Oacc,
                                                   int16_t* __restrict__ Oe, uint8_t* __restrict__ P, int T, int H, int D, int blk, int GA,
                                                   int kid) {
    __shared__ int qa[TMAX][4], ka[TMAX][4], va[TMAX][4];
    __shared__ int red[TMAX / 64];
    const int b = blockIdx.x / H, h = blockIdx.x % H, ld = 3 * D, b0 = b * T;
    int eq, ek, ev;
    alinha4<NR>(qm, qE, ld, h * 4, blk, b0, T, GA, red, qa, eq);
    alinha4<NR>(qm, qE, ld, D + h * 4, blk, b0, T, GA, red, ka, ek);
    alinha4<NR>(qm, qE, ld, 2 * D + h * 4, blk, b0, T, GA, red, va, ev);
    __syncthreads();
    const int su = -(eq + ek - 1 + 8), incl = 8 - h / 8;
    uint8_t* Pb = P + (size_t)blockIdx.x * T * T;
#pragma unroll 1
    for (int k = 0; k < NR; k++) {                                  // no barrier below: threads without a row leave
        const int i = linha_de<NR>(threadIdx.x, k, T), row = b0 + i;
        if (i < 0) continue;
        const int q0 = qa[i][0], q1 = qa[i][1], q2 = qa[i][2], q3 = qa[i][3];
        const long long idx = (long long)row * D + h * 4;
        auto sc = [&](int j) {
            const int s = mul24(q0, ka[j][0]) + mul24(q1, ka[j][1]) + mul24(q2, ka[j][2]) + mul24(q3, ka[j][3]);
            return rnd(s, su, kid, idx) - ((i - j) << incl);
        };
        int mx = U_MIN;
        for (int j = 0; j <= i; j++) mx = max(mx, sc(j));
        int soma = 0;
        for (int j = 0; j <= i; j++) soma += exp_dif(mx, sc(j)) >> 3;
        if (soma <= 0) { reporta(E_DIV, kid, idx, soma, mx); soma = 1; }
        const int inv = (1 << 28) / soma;
        int o[4] = {0, 0, 0, 0};
        for (int j = 0; j < T; j++) {
            int p = 0;
            if (j <= i) {
                const int ex = exp_dif(mx, sc(j)) >> 3;
                p = min((mul24(ex, inv) + (1 << 19)) >> 20, 255);
#pragma unroll
                for (int d = 0; d < 4; d++) o[d] += mul24(p, va[j][d]);
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
}

template <int TMAX, int LIMITE, int NR>
__global__ void __launch_bounds__(TMAX) k_atencao4_back(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE,
                                                        const int8_t* __restrict__ qm, const int8_t* __restrict__ qE,
                                                        const uint8_t* __restrict__ P, int* __restrict__ Gacc, int16_t* __restrict__ Ge,
                                                        int T, int H, int D, int blk, int GA, int DSB, int kid) {
    __shared__ int goa[TMAX][4], qa[TMAX][4], ka[TMAX][4], va[TMAX][4], slin[TMAX];
    __shared__ int red[TMAX / 64];
    const int b = blockIdx.x / H, h = blockIdx.x % H, ld = 3 * D, b0 = b * T;
    const uint8_t* Pb = P + (size_t)blockIdx.x * T * T;
    int eq, ek, ev, ego;
    alinha4<NR>(gom, goE, D, h * 4, blk, b0, T, GA, red, goa, ego);
    alinha4<NR>(qm, qE, ld, h * 4, blk, b0, T, GA, red, qa, eq);
    alinha4<NR>(qm, qE, ld, D + h * 4, blk, b0, T, GA, red, ka, ek);
    alinha4<NR>(qm, qE, ld, 2 * D + h * 4, blk, b0, T, GA, red, va, ev);
    __syncthreads();
    // the thread's rows (-1: none); every thread stays for the barriers of the block reductions
    int lin[NR];
#pragma unroll
    for (int k = 0; k < NR; k++) lin[k] = linha_de<NR>(threadIdx.x, k, T);
    auto gp_ij = [&](int i, int j) {
        return mul24(goa[i][0], va[j][0]) + mul24(goa[i][1], va[j][1]) + mul24(goa[i][2], va[j][2]) + mul24(goa[i][3], va[j][3]);
    };
    // shift of gP: exact causal maximum, or max_i ||dO_i||_inf * max_j ||v_j||_1
    int mg = 0;
    if constexpr (LIMITE) {
        int b1 = 0, b2 = 0;
#pragma unroll
        for (int k = 0; k < NR; k++) {
            const int i = lin[k];
            if (i < 0) continue;
            b1 = max(b1, max(max(abs(goa[i][0]), abs(goa[i][1])), max(abs(goa[i][2]), abs(goa[i][3]))));
            b2 = max(b2, abs(va[i][0]) + abs(va[i][1]) + abs(va[i][2]) + abs(va[i][3]));
        }
        mg = bloco_max(b1, red) * bloco_max(b2, red);
    } else {
#pragma unroll
        for (int k = 0; k < NR; k++)
            for (int j = 0; j <= lin[k]; j++) mg = max(mg, abs(gp_ij(lin[k], j)));
        mg = bloco_max(mg, red);
    }
    const int sh = max(bitlen(mg) - 15, 0), egp = ego + ev + sh;
    // s_i = rnd(sum_j P_ij gP'_ij, 8)
    int sl[NR], pm = 0, gm = 0;
#pragma unroll
    for (int k = 0; k < NR; k++) {
        const int i = lin[k];
        int s = 0;
        for (int j = 0; j <= i; j++) {
            const int p = Pb[(size_t)j * T + i], gp = rnd_d(gp_ij(i, j), sh);
            s += mul24(p, gp);
            if constexpr (LIMITE) { pm = max(pm, p); gm = max(gm, abs(gp)); }
        }
        if (s >= LIM || s <= -LIM) reporta(E_ACUM, kid, (long long)(b0 + i) * ld + h * 4, s, -4);
        sl[k] = rnd_d(s, 8);
        if (i >= 0) slin[i] = sl[k];
    }
    // shift of dS: exact maximum of |P (gP' - s)|, or max P * (max |gP'| + max |s|)
    int md = 0;
    if constexpr (LIMITE) {
        int sm = 0;
#pragma unroll
        for (int k = 0; k < NR; k++) sm = max(sm, lin[k] >= 0 ? abs(sl[k]) : 0);
        const int pmb = bloco_max(pm, red), gmb = bloco_max(gm, red), smb = bloco_max(sm, red);
        md = pmb * (gmb + smb);
    } else {
#pragma unroll
        for (int k = 0; k < NR; k++)
            for (int j = 0; j <= lin[k]; j++) md = max(md, abs(mul24((int)Pb[(size_t)j * T + lin[k]], rnd_d(gp_ij(lin[k], j), sh) - sl[k])));
        md = bloco_max(md, red);                                   // also publishes slin
    }
    const int sh2 = max(bitlen(md) - DSB, 0), eds = egp - 9 + sh2;
    // no barrier below: a thread without rows is done
#pragma unroll 1
    for (int k = 0; k < NR; k++) {
        const int i = lin[k];
        if (i < 0) continue;
        // row i: gq_i = sum_j dS_ij k_j
        int gq[4] = {0, 0, 0, 0};
        for (int j = 0; j <= i; j++) {
            const int ds = rnd_d(mul24((int)Pb[(size_t)j * T + i], rnd_d(gp_ij(i, j), sh) - sl[k]), sh2);
#pragma unroll
            for (int d = 0; d < 4; d++) gq[d] += mul24(ds, ka[j][d]);
        }
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const size_t o = (size_t)(b0 + i) * ld + h * 4 + d;
            if (gq[d] >= LIM || gq[d] <= -LIM) reporta(E_ACUM, kid, o, gq[d], -5);
            Gacc[o] = gq[d];
            Ge[o] = (int16_t)(eds + ek);
        }
        // column jj = i: gk_j = sum_{i >= j} dS_ij q_i, gv_j = sum_{i >= j} P_ij dO_i (row j of the stored P is contiguous)
        const int jj = i;
        const int v0 = va[jj][0], v1 = va[jj][1], v2 = va[jj][2], v3 = va[jj][3];
        const uint8_t* Pr = Pb + (size_t)jj * T;
        int gk[4] = {0, 0, 0, 0}, gv[4] = {0, 0, 0, 0};
        for (int ii = jj; ii < T; ii++) {
            const int p = Pr[ii];
            const int gp = mul24(goa[ii][0], v0) + mul24(goa[ii][1], v1) + mul24(goa[ii][2], v2) + mul24(goa[ii][3], v3);
            const int ds = rnd_d(mul24(p, rnd_d(gp, sh) - slin[ii]), sh2);
#pragma unroll
            for (int d = 0; d < 4; d++) { gk[d] += mul24(ds, qa[ii][d]); gv[d] += mul24(p, goa[ii][d]); }
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

// ---------------------------------------------------------------------------------------------- LPR lanes per row
// The same arithmetic with LPR consecutive lanes per query row (T <= TMAX = 128): lane l of row i takes the keys
// j = l, l + LPR, ... <= i and keeps their per-pair values in registers, so each score, exponential, gP and dS is
// computed once instead of once per pass; the row's maxima and sums combine across its LPR lanes (integer max and
// sum: exact in any order). LPR x the threads of one-row-per-thread, and the work of a row split LPR ways. A wave
// holds 64 / LPR consecutive rows, so the number of key steps it needs is known per wave (kr rows, kc columns):
// the unrolled steps past it are skipped by a scalar branch, and the causal half of the pairs costs nothing.
// The backward loads the head's whole P ([j][i] as stored) into LDS first with 16-byte accesses (rows 144 bytes
// apart: 16-byte aligned, and the 8 keys a wave touches at once fall on different banks) instead of reading one
// byte per pair twice. The forward writes P the same way round: a byte per pair into the head's transposed P in
// LDS, then 16-byte stores of whole rows.
constexpr int PLD = 144;
// the T x T bytes of global P ([j][i], rows of T) into the LDS copy (rows of PLD), 16 bytes per thread and step
__device__ __forceinline__ void carrega_p(const uint8_t* __restrict__ Pg, uint8_t (*ps)[PLD], int T) {
    const int porl = T / 16, n = T * porl;
    for (int c = threadIdx.x; c < n; c += blockDim.x) {
        const int r = c / porl, col = (c - r * porl) * 16;
        *reinterpret_cast<int4*>(&ps[r][col]) = *reinterpret_cast<const int4*>(Pg + (size_t)r * T + col);
    }
}
// carrega_p with at most CH chunks per thread (CH blockDim.x >= T T / 16), unrolled: a loop's head would wait for
// every load issued before it
template <int CH>
__device__ __forceinline__ void carrega_p_u(const uint8_t* __restrict__ Pg, uint8_t (*ps)[PLD], int T) {
    const int porl = T / 16, n = T * porl;
#pragma unroll
    for (int k = 0; k < CH; k++) {
        const int c = threadIdx.x + k * blockDim.x;
        if (c < n) {
            const int r = c / porl, col = (c - r * porl) * 16;
            *reinterpret_cast<int4*>(&ps[r][col]) = *reinterpret_cast<const int4*>(Pg + (size_t)r * T + col);
        }
    }
}
// NS head slices of 4 columns aligned at once (the alignment of alinha4<1>): thread t < T loads token t's 4 bytes
// and block exponent of every slice before anything waits, and one workgroup reduction gives all NS head maxima.
// entre() runs between those loads and the reduction: a copy into LDS placed there has its loads in flight with
// these (before them, its LDS store would wait for its own load before they are issued); the reduction's barrier
// publishes it.
struct Fatia4 { const int8_t *m, *E; int ld, col; };
template <int NS, int NW, class Entre>
__device__ __forceinline__ void alinha4n(const Fatia4 (&f)[NS], int blk, int b0, int T, int GA, int (&red)[NS][NW], int (*const (&al)[NS])[4],
                                         int (&eo)[NS], Entre&& entre) {
    const int t = threadIdx.x;
    int e[NS], w[NS], mx[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        e[s] = t < T ? (int)f[s].E[(size_t)(b0 + t) * (f[s].ld / blk) + f[s].col / blk] : SEM_TOPO;
        w[s] = t < T ? *reinterpret_cast<const int*>(f[s].m + (size_t)(b0 + t) * f[s].ld + f[s].col) : 0;
    }
    entre();
#pragma unroll
    for (int s = 0; s < NS; s++) mx[s] = g_max<64>(e[s]);
    if ((t & 63) == 0)
#pragma unroll
        for (int s = 0; s < NS; s++) red[s][t >> 6] = mx[s];
    __syncthreads();
#pragma unroll
    for (int s = 0; s < NS; s++) {
        int r = SEM_TOPO;
#pragma unroll
        for (int x = 0; x < NW; x++) r = max(r, red[s][x]);
        if (t < T)
#pragma unroll
            for (int d = 0; d < 4; d++) al[s][t][d] = rnd_d(((w[s] << (24 - 8 * d)) >> 24) << GA, r - e[s]);
        eo[s] = r - GA;
    }
}

template <int TMAX, int LPR>
__global__ void __launch_bounds__(TMAX * LPR) k_atencao4l(const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, int* __restrict__ Oacc,
                                                          int16_t* __restrict__ Oe, uint8_t* __restrict__ P, int T, int H, int D, int blk,
                                                          int GA, int kid) {
    constexpr int NJ = TMAX / LPR, NW = TMAX * LPR / 64;
    __shared__ int qa[TMAX][4], ka[TMAX][4], va[TMAX][4];
    __shared__ int red[3][NW];
    __shared__ __align__(16) unsigned short texp[EXP_N];
    __shared__ __align__(16) uint8_t pt[TMAX][PLD];                // P of the head, transposed ([j][i])
    static_assert(PLD >= TMAX && PLD % 16 == 0, "P rows in LDS");
    const int b = blockIdx.x / H, h = blockIdx.x % H, ld = 3 * D, b0 = b * T;
    int eo[3];
    {
        const Fatia4 f[3] = {{qm, qE, ld, h * 4}, {qm, qE, ld, D + h * 4}, {qm, qE, ld, 2 * D + h * 4}};
        int (*const al[3])[4] = {qa, ka, va};
        alinha4n<3, NW>(f, blk, b0, T, GA, red, al, eo, [&] { exp_tab_lds(texp); });
    }
    const int eq = eo[0], ek = eo[1], ev = eo[2];
    __syncthreads();
    const int su = __builtin_amdgcn_readfirstlane(-(eq + ek - 1 + 8)), incl = 8 - h / 8;   // one per head
    const int i = threadIdx.x / LPR, l = threadIdx.x % LPR;
    const bool ativo = i < T;
    const int ii = ativo ? i : 0, row = b0 + ii;
    const long long idx = (long long)row * D + h * 4;
    const int q0 = qa[ii][0], q1 = qa[ii][1], q2 = qa[ii][2], q3 = qa[ii][3];
    // key steps of this wave: its last row is min(T, 64 / LPR (w + 1)) - 1
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kr = __builtin_amdgcn_readfirstlane((min(T, (64 / LPR) * (w + 1)) - 1) / LPR + 1);
    // the ALiBi term (i - j) << incl of key j = l + LPR k is ab - k (LPR << incl) (shifts distribute over the
    // subtraction in 32-bit arithmetic); the score's rounding shift su is one per head: for su >= 0 one FMA (Desl,
    // exact for |score| < 2^26), a left shift (checked) otherwise
    const int ab = (ii - l) * (1 << incl), pa = LPR << incl;         // ii - l may be negative: no left shift of it
    const bool direita = su >= 0;
    const Desl dsu(su);
    int u[NJ], mx = U_MIN;
#pragma unroll
    for (int k = 0; k < NJ; k++) {
        const int j = l + LPR * k;
        if (k < kr && ativo && j <= i) {
            const int sc = mul24(q0, ka[j][0]) + mul24(q1, ka[j][1]) + mul24(q2, ka[j][2]) + mul24(q3, ka[j][3]);
            u[k] = (direita ? dsu(sc) : rnd(sc, su, kid, idx)) - ab + k * pa;
            mx = max(mx, u[k]);
        }
    }
    mx = g_max<LPR>(mx);
    int soma = 0;
#pragma unroll
    for (int k = 0; k < NJ; k++) {
        const int j = l + LPR * k;
        if (k < kr && ativo && j <= i) { u[k] = exp_tab(texp, mx, u[k]); soma += u[k]; }
    }
    soma = g_sum<LPR>(soma);
    if (ativo && soma <= 0) {
        if (l == 0) reporta(E_DIV, kid, idx, soma, mx);
        soma = 1;
    }
    // a row's sum is at least 4095 (its maximum contributes exp(0) >> 3), so 2^28 / sum < 2^20: div_exata's bound
    const int inv = soma > 256 ? div_exata(1 << 28, soma) : (1 << 28) / max(soma, 1);
    uint8_t* Pb = P + (size_t)blockIdx.x * T * T;
    int o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < NJ; k++) {
        const int j = l + LPR * k;
        int p = 0;
        if (k < kr && ativo && j <= i) {
            p = min((mul24(u[k], inv) + (1 << 19)) >> 20, 255);
#pragma unroll
            for (int d = 0; d < 4; d++) o[d] += mul24(p, va[j][d]);
        }
        if (ativo && j < T) pt[j][i] = (uint8_t)p;
    }
#pragma unroll
    for (int d = 0; d < 4; d++) o[d] = g_sum<LPR>(o[d]);
    // the head's P, transposed in LDS, goes out as 16-byte pieces of whole rows: byte stores scattered over rows T
    // apart cost 7.7 of this kernel's 27 us at the reference shape, these 2.5
    __syncthreads();
    {
        const int porl = T / 16, n = T * porl;
        for (int c = threadIdx.x; c < n; c += blockDim.x) {
            const int r = c / porl, col = (c - r * porl) * 16;
            *reinterpret_cast<int4*>(Pb + (size_t)r * T + col) = *reinterpret_cast<const int4*>(&pt[r][col]);
        }
    }
    if (!ativo || l != 0) return;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const size_t x = (size_t)row * D + h * 4 + d;
        if (o[d] >= LIM || o[d] <= -LIM) reporta(E_ACUM, kid, x, o[d], -3);
        Oacc[x] = o[d];
        Oe[x] = (int16_t)(ev - 8);
    }
}

// Backward with LPR lanes per row. Rows: lane l of row i keeps gP'_ij, P_ij and then dS_ij for its keys in
// registers and writes dS to LDS ([i][j], int16: |dS| < 2^DSB <= 2^12). Columns: lane l of column j sums over the
// rows i = j + l, j + l + LPR, ... < T, reading dS from LDS and P from its contiguous stored row.
template <int TMAX, int LIMITE, int LPR>
__global__ void __launch_bounds__(TMAX * LPR) k_atencao4l_back(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE,
                                                               const int8_t* __restrict__ qm, const int8_t* __restrict__ qE,
                                                               const uint8_t* __restrict__ P, int* __restrict__ Gacc, int16_t* __restrict__ Ge,
                                                               int T, int H, int D, int blk, int GA, int DSB, int kid) {
    constexpr int NJ = TMAX / LPR, LDS_ = TMAX + 2, NW = TMAX * LPR / 64;
    __shared__ int goa[TMAX][4], qa[TMAX][4], ka[TMAX][4], va[TMAX][4];
    __shared__ int16_t dsm[TMAX][LDS_];
    __shared__ int red[TMAX * LPR / 64];
    __shared__ int red4[4][NW];
    __shared__ __align__(16) uint8_t ps[TMAX][PLD];
    const int b = blockIdx.x / H, h = blockIdx.x % H, ld = 3 * D, b0 = b * T;
    const uint8_t* Pb = P + (size_t)blockIdx.x * T * T;
    int eo[4];
    {
        const Fatia4 f[4] = {{gom, goE, D, h * 4}, {qm, qE, ld, h * 4}, {qm, qE, ld, D + h * 4}, {qm, qE, ld, 2 * D + h * 4}};
        int (*const al[4])[4] = {goa, qa, ka, va};
        alinha4n<4, NW>(f, blk, b0, T, GA, red4, al, eo, [&] { carrega_p_u<(TMAX * TMAX / 16 + TMAX * LPR - 1) / (TMAX * LPR)>(Pb, ps, T); });
    }
    const int ego = eo[0], eq = eo[1], ek = eo[2], ev = eo[3];
    __syncthreads();
    const int i = threadIdx.x / LPR, l = threadIdx.x % LPR;
    const bool ativo = i < T;
    const int ii = ativo ? i : 0;
    const int g0 = goa[ii][0], g1 = goa[ii][1], g2 = goa[ii][2], g3 = goa[ii][3];
    // key steps of this wave as rows (its last row is min(T, 64 / LPR (w + 1)) - 1) and as columns (its first
    // column is 64 / LPR w)
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kr = __builtin_amdgcn_readfirstlane((min(T, (64 / LPR) * (w + 1)) - 1) / LPR + 1);
    const int kc = __builtin_amdgcn_readfirstlane(max(T - (64 / LPR) * w, 0) / LPR + 1);
    // gP_ij = dO_i . v_j and P_ij of the lane's keys
    int gp[NJ], pp[NJ];
    int mg = 0;
#pragma unroll
    for (int k = 0; k < NJ; k++) {
        const int j = l + LPR * k;
        if (k < kr && ativo && j <= i) {
            gp[k] = mul24(g0, va[j][0]) + mul24(g1, va[j][1]) + mul24(g2, va[j][2]) + mul24(g3, va[j][3]);
            pp[k] = ps[j][i];
            if constexpr (!LIMITE) mg = max(mg, abs(gp[k]));
        }
    }
    // shift of gP: exact causal maximum, or max_i ||dO_i||_inf * max_j ||v_j||_1
    if constexpr (LIMITE) {
        const int b1 = ativo ? max(max(abs(g0), abs(g1)), max(abs(g2), abs(g3))) : 0;
        const int b2 = ativo ? abs(va[i][0]) + abs(va[i][1]) + abs(va[i][2]) + abs(va[i][3]) : 0;
        mg = bloco_max(b1, red) * bloco_max(b2, red);
    } else {
        mg = bloco_max(mg, red);
    }
    const int sh = max(bitlen(mg) - 15, 0), egp = ego + ev + sh;
    // s_i = rnd(sum_j P_ij gP'_ij, 8)
    int s = 0, pm = 0, gm = 0;
#pragma unroll
    for (int k = 0; k < NJ; k++) {
        const int j = l + LPR * k;
        if (k < kr && ativo && j <= i) {
            gp[k] = rnd_d(gp[k], sh);
            s += mul24(pp[k], gp[k]);
            if constexpr (LIMITE) { pm = max(pm, pp[k]); gm = max(gm, abs(gp[k])); }
        }
    }
    s = g_sum<LPR>(s);
    if (ativo && l == 0 && (s >= LIM || s <= -LIM)) reporta(E_ACUM, kid, (long long)(b0 + i) * ld + h * 4, s, -4);
    const int sl = rnd_d(s, 8);
    // shift of dS: exact maximum of |P (gP' - s)|, or max P * (max |gP'| + max |s|)
    int md = 0;
    if constexpr (LIMITE) {
        const int pmb = bloco_max(pm, red), gmb = bloco_max(gm, red), smb = bloco_max(ativo ? abs(sl) : 0, red);
        md = pmb * (gmb + smb);
    } else {
#pragma unroll
        for (int k = 0; k < NJ; k++) {
            const int j = l + LPR * k;
            if (k < kr && ativo && j <= i) md = max(md, abs(mul24(pp[k], gp[k] - sl)));
        }
        md = bloco_max(md, red);
    }
    const int sh2 = max(bitlen(md) - DSB, 0), eds = egp - 9 + sh2;
    // row i: dS_ij to LDS, gq_i = sum_j dS_ij k_j
    int gq[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < NJ; k++) {
        const int j = l + LPR * k;
        if (k < kr && ativo && j <= i) {
            const int ds = rnd_d(mul24(pp[k], gp[k] - sl), sh2);
            dsm[i][j] = (int16_t)ds;
#pragma unroll
            for (int d = 0; d < 4; d++) gq[d] += mul24(ds, ka[j][d]);
        }
    }
#pragma unroll
    for (int d = 0; d < 4; d++) gq[d] = g_sum<LPR>(gq[d]);
    if (ativo && l == 0) {
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const size_t o = (size_t)(b0 + i) * ld + h * 4 + d;
            if (gq[d] >= LIM || gq[d] <= -LIM) reporta(E_ACUM, kid, o, gq[d], -5);
            Gacc[o] = gq[d];
            Ge[o] = (int16_t)(eds + ek);
        }
    }
    __syncthreads();                                                 // every dS of the head in LDS
    // column j = i: gk_j = sum_{r >= j} dS_rj q_r, gv_j = sum_{r >= j} P_rj dO_r (row j of the stored P is contiguous)
    const int j = ii;
    const uint8_t* Pr = ps[j];
    int gk[4] = {0, 0, 0, 0}, gv[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < NJ; k++) {
        const int r = j + l + LPR * k;
        if (k < kc && ativo && r < T) {
            const int ds = dsm[r][j], p = Pr[r];
#pragma unroll
            for (int d = 0; d < 4; d++) { gk[d] += mul24(ds, qa[r][d]); gv[d] += mul24(p, goa[r][d]); }
        }
    }
#pragma unroll
    for (int d = 0; d < 4; d++) { gk[d] = g_sum<LPR>(gk[d]); gv[d] = g_sum<LPR>(gv[d]); }
    if (!ativo || l != 0) return;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const size_t o = (size_t)(b0 + j) * ld + h * 4 + d;
        if (gk[d] >= LIM || gk[d] <= -LIM) reporta(E_ACUM, kid, o + D, gk[d], -5);
        if (gv[d] >= LIM || gv[d] <= -LIM) reporta(E_ACUM, kid, o + 2 * D, gv[d], -5);
        Gacc[o + D] = gk[d];
        Ge[o + D] = (int16_t)(eds + eq);
        Gacc[o + 2 * D] = gv[d];
        Ge[o + 2 * D] = (int16_t)(ego - 8);
    }
}
