// Causal ALiBi attention at head width 64 with a caller-provided workspace (the arithmetic of k_atencao_mf: the
// declared head-width-64 generalization of ops.py:186-258).
//
// Forward in two launches:
//   (1) k_atf_prep, one workgroup per (sequence, head, 64 tokens): the head-wide exponent maxima of q, k, v (one
//       pass, one reduction), k as m8 << L fragments (int8 [T][64] + L [T][2]) and v aligned as f16 in the order
//       k_atf's PV MFMAs read it, into the workspace -- converted once instead of once per query block;
//   (2) k_atf, one workgroup of 4 waves per (sequence, head, 16 query rows): wave w takes the key tiles
//       t = w, w + 4, ... up to the diagonal. The row maxima and row sums combine across the waves through LDS
//       (integer max and sum: exact in any order); each wave multiplies its P tiles by V on f16 MFMA, and the
//       four partial outputs are added in fp32: every partial and their sum are integers below 2^20 (P <= 255,
//       |v| <= 2032, a row of P sums to at most 256 + T/2), so the sum is exact and equals the one-pass result.
// 4096 waves at config 4 (4 per SIMD) instead of 1024, each with a quarter of the serial score/softmax chain.
// The scalar products are 24-bit ones (mul24): P <= 255, ex <= 4095 and 2^28 / sum ex <= 2^16 (the row maximum
// alone adds 4095 to the sum), |gP'| <= 2^15 and |gP' - s| < 2^17 (a row of P sums to at most 256 + T / 2).
#include "jt_comum.h"

constexpr size_t cmax_(size_t a, size_t b) { return a > b ? a : b; }

namespace atw {
// workspace parts, each 256-byte aligned: km8 int8 [BH][T][64]; kl int8 [BH][T][2]; vf f16 [BH][NPV(T)][4][64][8];
// mx int [BH][4] (emq, emk, emv).
// km8 rows hold the 8-byte chunks of dimensions 8 k .. 8 k + 7 at chunk 2 (k % 4) + k / 4, so a lane's two MFMA
// fragments of a key (dimensions 8 g .. and 32 + 8 g ..) are one 16-byte load and a wave's 16 keys one kilobyte.
// vf holds v as the PV MFMAs' B fragments: slot p pairs the key tiles ta = 8 (p / 4) + p % 4 and ta + 4; its
// block for dimension group dt is 64 lanes x 8 values, lane 16 lg + lr holding dimension 16 dt + lr of the keys
// 16 (lg < 2 ? ta : ta + 4) + 8 (lg % 2) .. + 7, so each of a wave's fragment loads reads one contiguous
// kilobyte. A half past the last key tile is never written: k_atf reads zeros there instead.
struct Ws {
    int8_t *km8, *kl;
    _Float16* vf;
    int* mx;
};
__host__ __device__ inline int npv(int T) { return 4 * ((T / 16 + 7) / 8); }       // slots of vf per head
__device__ __forceinline__ int pos_k8(int k) { return 2 * (k & 3) + (k >> 2); }     // km8 chunk position of chunk k
inline size_t alinha256(size_t n) { return (n + 255) & ~(size_t)255; }
inline size_t bytes_fwd(long long BH, int T) {
    const size_t n = (size_t)BH * T;
    return alinha256(n * 64) + alinha256(n * 2) + alinha256((size_t)BH * npv(T) * 4096) + alinha256((size_t)BH * 16);
}
inline Ws parte(void* base, long long BH, int T) {
    const size_t n = (size_t)BH * T;
    char* p = (char*)base;
    Ws w;
    w.km8 = (int8_t*)p; p += alinha256(n * 64);
    w.kl = (int8_t*)p; p += alinha256(n * 2);
    w.vf = (_Float16*)p; p += alinha256((size_t)BH * npv(T) * 4096);
    w.mx = (int*)p;
    return w;
}
// The backward's conversions of q, k, v, written by the forward's conversion pass, which has those values loaded
// (kept by the caller from the forward to the backward of the same qkv): vm8 int8 [BH][T][64] (chunks as km8's);
// vL int8 [BH][T][2]; kt, qt f16 [BH][64][T] in fragment order (grava_ft64); mx int [BH][4] (emq, emk, emv: the
// head maxima, before - GA)
struct Salvo {
    int8_t *vm8, *vL;
    _Float16 *kt, *qt;
    int* mx;
};
inline size_t bytes_salvo(long long BH, int T) {
    const size_t n = (size_t)BH * T;
    return alinha256(n * 64) + alinha256(n * 2) + 2 * alinha256(n * 64 * 2) + alinha256((size_t)BH * 16);
}
inline Salvo parte_s(void* base, long long BH, int T) {
    const size_t n = (size_t)BH * T;
    char* p = (char*)base;
    Salvo s;
    s.vm8 = (int8_t*)p; p += alinha256(n * 64);
    s.vL = (int8_t*)p; p += alinha256(n * 2);
    s.kt = (_Float16*)p; p += alinha256(n * 64 * 2);
    s.qt = (_Float16*)p; p += alinha256(n * 64 * 2);
    s.mx = (int*)p;
    return s;
}
}

// Largest block exponent of the 64 / blk blocks of a head slice in one token's exponent row e (column c0): at
// BLK = 32 the slice's two bytes in one 2-byte load (c0 / 32 is even), at BLK = 128 its one byte.
__device__ __forceinline__ int emx_fatia(const int8_t* e, int c0, int blk) {
    if (blk == 32) {
        const int x = *reinterpret_cast<const short*>(e + c0 / 32);
        return max((int)(int8_t)x, x >> 8);
    }
    return (int)e[c0 / blk];
}

// Largest block exponents of three head slices (columns c0 + [0, 64) of E, one per slice) over the T tokens of
// sequence b0 / T: one token per thread (T <= 512: at most two), one workgroup reduction (256 threads).
__device__ __forceinline__ void emx3(const int8_t* E, int ld, int ca, int cb, int cc, int blk, int b0, int T, int (&red)[3][4], int& a, int& b,
                                     int& c) {
    const int nbl = ld / blk;
    int ma = SEM_TOPO, mb = SEM_TOPO, mc = SEM_TOPO;
    for (int t = threadIdx.x; t < T; t += 256) {
        const int8_t* e = E + (size_t)(b0 + t) * nbl;
        ma = max(ma, emx_fatia(e, ca, blk)); mb = max(mb, emx_fatia(e, cb, blk)); mc = max(mc, emx_fatia(e, cc, blk));
    }
    ma = g_max<64>(ma); mb = g_max<64>(mb); mc = g_max<64>(mc);
    if ((threadIdx.x & 63) == 0) { red[0][threadIdx.x >> 6] = ma; red[1][threadIdx.x >> 6] = mb; red[2][threadIdx.x >> 6] = mc; }
    __syncthreads();
    a = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
    b = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));
    c = max(max(red[2][0], red[2][1]), max(red[2][2], red[2][3]));
}

// The workgroup's 64 tokens x 64 dimensions of a transposed f16 array ([BH][64][T]), staged in LDS by the threads
// that converted them, written out as 16-byte chunks of each dimension's 128-byte row segment (two per thread)
// instead of sixteen scattered 2-byte stores per thread. Call after a barrier that follows the tile's writes.
typedef _Float16 TileT[64][72];                                      // rows padded to 144 bytes (16-byte aligned)
__device__ __forceinline__ void grava_t64(const TileT& tile, _Float16* __restrict__ cab, int T, int t0) {
#pragma unroll
    for (int x = threadIdx.x; x < 64 * 8; x += 256) {
        const int row = x >> 3, ch = x & 7;
        *reinterpret_cast<int4*>(cab + (size_t)row * T + t0 + 8 * ch) = *reinterpret_cast<const int4*>(&tile[row][8 * ch]);
    }
}
// The same 64 tokens x 64 dimensions (key tiles 4 p .. 4 p + 3 of a head, p = t0 / 64) in fragment order, the
// head's [64][T] f16 array as [T / 16 tiles][4 dt][2 h][16 lr][8]: lane (lr, lg) of an f16 MFMA B fragment reading
// dimension 16 dt + lr of keys 16 t + 8 h .. + 7 (h = lg % 2) finds them at block (t, dt, h), row lr, so the 32
// lanes of one tile read 512 contiguous bytes, where [64][T] rows gave them 32-byte pieces of 16 rows.
__device__ __forceinline__ size_t pos_ft(int t, int dt, int h, int lr) { return ((((size_t)t * 4 + dt) * 2 + h) * 16 + lr) * 8; }
__device__ __forceinline__ void grava_ft64(const TileT& tile, _Float16* __restrict__ cab, int t0) {
    const int x = threadIdx.x, i = x >> 6, dt = (x >> 4) & 3, lr = x & 15, t = t0 / 16 + i;
#pragma unroll
    for (int h = 0; h < 2; h++)
        *reinterpret_cast<int4*>(cab + pos_ft(t, dt, h, lr)) = *reinterpret_cast<const int4*>(&tile[16 * dt + lr][16 * i + 8 * h]);
}
// 16 m8 values of a token's dimensions 16 c4 .. 16 c4 + 15 into its 64-byte row with the 8-byte chunks k at
// 2 (k % 4) + k / 4 (atw::pos_k8), so an MFMA lane's two fragments (dimensions 8 g .. and 32 + 8 g ..) are one
// 16-byte load
__device__ __forceinline__ void grava_m8_fragmentos(int8_t* __restrict__ linha, int c4, const int8_t (&m8)[16]) {
    int8_t lo[8], hi[8];
#pragma unroll
    for (int k = 0; k < 8; k++) { lo[k] = m8[k]; hi[k] = m8[8 + k]; }
    grava_i8(linha + 8 * atw::pos_k8(2 * c4), lo);
    grava_i8(linha + 8 * atw::pos_k8(2 * c4 + 1), hi);
}
// the two fragments (chunks g and 4 + g) of a row written that way
__device__ __forceinline__ void le_m8_fragmentos(const int8_t* __restrict__ linha, int g, long& f0, long& f1) {
    const int4 x = *reinterpret_cast<const int4*>(linha + 16 * g);
    f0 = (long)(unsigned)x.x | ((long)x.y << 32);
    f1 = (long)(unsigned)x.z | ((long)x.w << 32);
}

// SALVA: also the backward's conversions of q, k, v into s (the arithmetic of k_atb_prep's: v as m8 << L
// fragments, q and k aligned as f16 [64][T], the head maxima), so the backward converts only dO.
template <bool SALVA = false>
__global__ void __launch_bounds__(256) k_atf_prep(const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, atw::Ws w, atw::Salvo s, int T,
                                                  int H, int D, int blk, int GA) {
    constexpr int HD = 64;
    __shared__ int red[3][4];
    __shared__ __align__(16) TileT tv;
    __shared__ __align__(16) TileT tqk[SALVA ? 2 : 1];              // SALVA: q and k aligned, for the backward
    const int nparts = T / 64, bh = blockIdx.x / nparts, part = blockIdx.x % nparts, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, nbl = ld / blk, tid = threadIdx.x;
    // thread (t, c4): dimensions 16 c4 .. 16 c4 + 15 of token t; its k and v values (and q with SALVA) are loaded
    // before the head maxima's barrier, so their latency overlaps it
    const int t = part * 64 + (tid >> 2), c4 = tid & 3, half = c4 >> 1;
    const size_t base = (size_t)(b0 + t) * ld, tt = (size_t)bh * T + t;
    const int colq = h * HD + 16 * c4, colk = D + colq, colv = 2 * D + colq;
    const int4 rk = ld16(qm + base + colk), rv = ld16(qm + base + colv);
    const int ekt = qE[(size_t)(b0 + t) * nbl + colk / blk], evt = qE[(size_t)(b0 + t) * nbl + colv / blk];
    int4 rq = make_int4(0, 0, 0, 0);
    int eqt = 0;
    if constexpr (SALVA) {
        rq = ld16(qm + base + colq);
        eqt = qE[(size_t)(b0 + t) * nbl + colq / blk];
    }
    int emq, emk, emv;
    emx3(qE, ld, h * HD, D + h * HD, 2 * D + h * HD, blk, b0, T, red, emq, emk, emv);
    if (part == 0 && tid == 0) {
        w.mx[bh * 4] = emq; w.mx[bh * 4 + 1] = emk; w.mx[bh * 4 + 2] = emv;
        if constexpr (SALVA) { s.mx[bh * 4] = emq; s.mx[bh * 4 + 1] = emk; s.mx[bh * 4 + 2] = emv; }
    }
    {
        int v[16];
        abre_i8(rk, v);
        const int sh = emk - ekt;
        int8_t m8[16];
        int L = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) { int a; m8_L(v[k], sh, GA, a, L); m8[k] = (int8_t)a; }
        grava_m8_fragmentos(w.km8 + tt * 64, c4, m8);
        if ((c4 & 1) == 0) w.kl[tt * 2 + half] = (int8_t)L;
        if constexpr (SALVA) {
            const Desl dk(emk - ekt);
#pragma unroll
            for (int k = 0; k < 16; k++) tqk[SALVA ? 1 : 0][16 * c4 + k][tid >> 2] = (_Float16)dk(shl(v[k], GA));
        }
    }
    {
        int v[16];
        abre_i8(rv, v);
        const Desl dv(emv - evt);                                    // rnd(v << GA, emv - evt), one shift per block
#pragma unroll
        for (int k = 0; k < 16; k++) tv[16 * c4 + k][tid >> 2] = (_Float16)dv(shl(v[k], GA));
        if constexpr (SALVA) {
            const int sh = emv - evt;
            int8_t m8[16];
            int L = 0;
#pragma unroll
            for (int k = 0; k < 16; k++) { int a; m8_L(v[k], sh, GA, a, L); m8[k] = (int8_t)a; }
            grava_m8_fragmentos(s.vm8 + tt * 64, c4, m8);
            if ((c4 & 1) == 0) s.vL[tt * 2 + half] = (int8_t)L;
        }
    }
    if constexpr (SALVA) {
        int v[16];
        abre_i8(rq, v);
        const Desl dq(emq - eqt);
#pragma unroll
        for (int k = 0; k < 16; k++) tqk[0][16 * c4 + k][tid >> 2] = (_Float16)dq(shl(v[k], GA));
    }
    __syncthreads();
    {   // v fragments of the part's 4 key tiles: thread x writes dimension 16 dt + lr of tile 4 part + x / 64, the
        // 8-key halves (lg % 2 = 0, 1) of its fragment block
        const int i = tid >> 6, dt = (tid >> 4) & 3, lr = tid & 15, tk = 4 * part + i;
        const int slot = 4 * (tk >> 3) + (tk & 3), meio = (tk >> 2) & 1;   // meio 1: the pair's second tile (lg >= 2)
        _Float16* dst = w.vf + ((((size_t)bh * atw::npv(T) + slot) * 4 + dt) * 64 + 32 * meio + lr) * 8;
#pragma unroll
        for (int h2 = 0; h2 < 2; h2++)
            *reinterpret_cast<int4*>(dst + 16 * 8 * h2) = *reinterpret_cast<const int4*>(&tv[16 * dt + lr][16 * i + 8 * h2]);
    }
    if constexpr (SALVA) {
        grava_ft64(tqk[0], s.qt + (size_t)bh * 64 * T, part * 64);
        grava_ft64(tqk[SALVA ? 1 : 0], s.kt + (size_t)bh * 64 * T, part * 64);
    }
}

// NTW = key tiles a wave can own (T / 64)
// Outputs of 16 rows x the head's 64 columns in block format (BLK = 32: two blocks per row): thread t holds row
// t / 16, columns 4 (t % 16) .. + 3; the 8 lanes of a block are consecutive. Same result as quant of the raw
// output (ops.py:125-126) with the block's common exponent e.
template <bool NT = true>
__device__ __forceinline__ void grava_bloco4(const int (&v)[4], int e, int8_t* __restrict__ Mm, int8_t* __restrict__ ME, size_t x, size_t xe,
                                             int kid) {
    int8_t q[4];
    const int E = quant8_u8<4, 8>(v, e, q, kid, (long long)x);
    grava_i8<4, NT>(Mm + x, q);
    if ((threadIdx.x & 7) == 0) ME[xe] = (int8_t)E;
}

// BLOCO: the output in block format (Oacc, Oe are then the mantissas and exponents, int8) instead of raw
template <int NTW, bool BLOCO = false>
__global__ void __launch_bounds__(256) k_atf(const int8_t* __restrict__ qm, const int8_t* __restrict__ qE, atw::Ws w, void* __restrict__ Oacc_,
                                             void* __restrict__ Oe_, uint8_t* __restrict__ P, int T, int H, int D, int blk, int GA, int kid) {
    constexpr int HD = 64, LP = 16 * (NTW + 1);                     // LDS row length of a wave's P (one pad tile)
    __shared__ int sred[4][16];
    __shared__ __align__(16) _Float16 pw[4][16][LP];
    __shared__ float so[4][16][68];                                  // rows of 68: rows 4 apart fall in other banks
    __shared__ __align__(16) unsigned short texp[EXP_N];
    static_assert(256 * 2 >= EXP_N / 8 && 256 <= EXP_N / 8, "exp table: one or two chunks per thread");
    int4 tch[2];
    exp_tab_le(tch);                                                 // into LDS once every other load is issued
    // workgroups in decreasing work across all heads (the query tile qt costs qt + 1 key tiles): the ones resident
    // together on a CU then mix long and short rows
    const int nqt = T / 16, BH = gridDim.x / nqt, bh = blockIdx.x % BH, qt = nqt - 1 - (int)(blockIdx.x / BH);
    const int b = bh / H, h = bh % H, b0 = b * T;
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lr = lane & 15, lg = lane >> 4;
    const int eq = w.mx[bh * 4] - GA, ek = w.mx[bh * 4 + 1] - GA, ev = w.mx[bh * 4 + 2] - GA;
    const int su = -(eq + ek - 3 + 8), incl = 8 - (8 * h) / H;     // log2(64) / 2 = 3
    const size_t hb = (size_t)bh * T;
    const int ia = 16 * qt + lr, i0 = 16 * qt + 4 * lg;              // A-fragment row; this lane's 4 score rows
    const int nv = qt >= wv ? (qt - wv) / 4 + 1 : 0;                 // this wave's key tiles wv + 4 n, n < nv
    // V fragments of the PV pairs, loaded first (they depend on nothing): pair m, k-index kk = 8 lg + e is key
    // 16 (wv + 4 (2m + kk / 16)) + kk % 16; a pad tile (P = 0 there) reads the wave's first tile of V
    constexpr int NPAR = (NTW + 1) / 2;
    h8_t vb[NPAR][4];
    // Buffer loads over the head's regions, every one issued (no branch between them): an offset past a region
    // (0x80000000) returns 0 and touches no memory, for a pair or tile the wave does not use and for V past the
    // last key tile (P = 0 and v = 0 there)
    const auto rsV = __builtin_amdgcn_make_buffer_rsrc((void*)(w.vf + (size_t)bh * atw::npv(T) * 2048), (short)0, atw::npv(T) * 4096, 0x00020000);
    const auto rsK = __builtin_amdgcn_make_buffer_rsrc((void*)(w.km8 + hb * 64), (short)0, T * 64, 0x00020000);
#pragma unroll
    for (int m = 0; m < NPAR; m++) {                                 // the slot of pair m is 4 m + wv
        const int tv = wv + 4 * (2 * m + (lg >> 1));
        const int off = 2 * m < nv && tv < nqt ? ((4 * m + wv) * 4 * 64 + lane) * 16 : (int)0x80000000;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            const v4i x = __builtin_amdgcn_raw_buffer_load_b128(rsV, off + dt * 64 * 16, 0, 0);
            vb[m][dt] = __builtin_bit_cast(h8_t, x);
        }
    }
    // K fragments of this wave's key tiles, loaded at entry as well
    long kb[NTW][2];
    unsigned lkr[NTW];                                                // both L bytes of a key, split where used
#pragma unroll
    for (int n = 0; n < NTW; n++) {                                   // a tile the wave does not own: 0 (its L
        const int jl = 16 * (n < nv ? wv + 4 * n : wv) + lr;          // bytes re-read from its first tile)
        const v4i x = __builtin_amdgcn_raw_buffer_load_b128(rsK, n < nv ? jl * 64 + 16 * lg : (int)0x80000000, 0, 0);
        kb[n][0] = (long)(unsigned)x[0] | ((long)x[1] << 32);        // le_m8_fragmentos' two fragments
        kb[n][1] = (long)(unsigned)x[2] | ((long)x[3] << 32);
        lkr[n] = *reinterpret_cast<const unsigned short*>(w.kl + (hb + jl) * 2);
    }
    // q fragments of the tile's 16 rows, converted here: A row lr = query ia, dimensions 32 c + 8 lg .. + 7
    __shared__ int qL[16][2];
    long qa[2];
    int qv[2][8], qe[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {                                     // both halves' loads before either conversion
        const int col = h * HD + 32 * c + 8 * lg;                     // (m8L_frag's arithmetic)
        le_i8(qm + (size_t)(b0 + ia) * (3 * D) + col, qv[c]);
        qe[c] = qE[(size_t)(b0 + ia) * (3 * D / blk) + col / blk];
    }
    exp_tab_grava(texp, tch);                                        // waits for the table's load only
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int s = eq + GA - qe[c];
        int L = 0;
        long pk = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) { int a; m8_L(qv[c][k], s, GA, a, L); pk |= (long)(uint8_t)a << (8 * k); }
        qa[c] = pk;
        if (lg == 0) qL[lr][c] = L;
    }
    __syncthreads();
    int lq[4][2];
#pragma unroll
    for (int v = 0; v < 4; v++) { lq[v][0] = qL[4 * lg + v][0]; lq[v][1] = qL[4 * lg + v][1]; }
    const long long idx = (long long)(b0 + i0) * D + h * HD;
    const Desl dsu(su);                                              // the scores' rounding shift, one per head
    int uu[NTW][4], mx[4] = {U_MIN, U_MIN, U_MIN, U_MIN};
#pragma unroll
    for (int n = 0; n < NTW; n++) {
        if (n >= nv) continue;                                       // guarded, not break: uu stays in registers
        const int j = 16 * (wv + 4 * n) + lr;
        const int lk0 = (int)(int8_t)(lkr[n] & 0xff), lk1 = (int)(int8_t)(lkr[n] >> 8);
        const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa[0], kb[n][0], v4i{0, 0, 0, 0}, 0, 0, 0);
        const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa[1], kb[n][1], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int i = i0 + v;
            const int s = shl(p0[v], lq[v][0] + lk0) + shl(p1[v], lq[v][1] + lk1);
            const int r = su >= 0 ? dsu(s) : rnd(s, su, kid, idx);
            const int u = j <= i ? r - ((i - j) << incl) : U_MIN;
            uu[n][v] = u;
            mx[v] = max(mx[v], u);
        }
    }
#pragma unroll
    for (int v = 0; v < 4; v++) mx[v] = g_max<16>(mx[v]);
    if (lr == 0)
#pragma unroll
        for (int v = 0; v < 4; v++) sred[wv][4 * lg + v] = mx[v];
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 4; v++) mx[v] = max(max(sred[0][4 * lg + v], sred[1][4 * lg + v]), max(sred[2][4 * lg + v], sred[3][4 * lg + v]));
    __syncthreads();                                                 // sred is reused for the sums
    int soma[4] = {0, 0, 0, 0};
#pragma unroll
    for (int n = 0; n < NTW; n++) {
        if (n >= nv) continue;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int ex = exp_tab(texp, mx[v], uu[n][v]);          // a masked pair (U_MIN) reads the final 0
            uu[n][v] = ex;
            soma[v] += ex;
        }
    }
#pragma unroll
    for (int v = 0; v < 4; v++) soma[v] = g_sum<16>(soma[v]);
    if (lr == 0)
#pragma unroll
        for (int v = 0; v < 4; v++) sred[wv][4 * lg + v] = soma[v];
    __syncthreads();
    int inv[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        int s = sred[0][4 * lg + v] + sred[1][4 * lg + v] + sred[2][4 * lg + v] + sred[3][4 * lg + v];
        if (s <= 0) { if (lr == 0 && wv == 0) reporta(E_DIV, kid, idx + (long long)v * D, s, mx[v]); s = 1; }
        // s >= 4095 (the row maximum contributes exp(0) >> 3), so 2^28 / s < 2^20: div_exata's bound
        inv[v] = s > 256 ? div_exata(1 << 28, s) : (1 << 28) / s;
    }
    uint8_t* Pb = P + (size_t)bh * T * T;
#pragma unroll
    for (int n = 0; n < NTW; n++) {
        if (n >= nv) continue;
        const int j = 16 * (wv + 4 * n) + lr;
        unsigned pk = 0;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int p = min((mul24(uu[n][v], inv[v]) + (1 << 19)) >> 20, 255);
            pk |= (unsigned)p << (8 * v);
            pw[wv][4 * lg + v][16 * n + lr] = (_Float16)p;
        }
        *reinterpret_cast<unsigned*>(Pb + (size_t)j * T + i0) = pk;
    }
    for (int t = wv + 4 * nv; t < nqt; t += 4) *reinterpret_cast<unsigned*>(Pb + (size_t)(16 * t + lr) * T + i0) = 0u;   // above the diagonal
    if (nv & 1)
#pragma unroll
        for (int v = 0; v < 4; v++) pw[wv][4 * lg + v][16 * nv + lr] = (_Float16)0;
    __syncthreads();
    // partial O = P V over this wave's tiles, in pairs
    f4_t o[4] = {};
#pragma unroll
    for (int m = 0; m < NPAR; m++) {
        if (2 * m >= nv) continue;
        const h8_t a = *reinterpret_cast<const h8_t*>(&pw[wv][lr][32 * m + 8 * lg]);
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, vb[m][dt], o[dt], 0, 0, 0);
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) so[wv][4 * lg + v][16 * dt + lr] = o[dt][v];
    __syncthreads();
    if constexpr (BLOCO) {
        const int r = tid >> 4, c = 4 * (tid & 15);
        int ov[4];
        const size_t x = (size_t)(b0 + 16 * qt + r) * D + h * HD + c;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            ov[k] = (int)(so[0][r][c + k] + so[1][r][c + k] + so[2][r][c + k] + so[3][r][c + k]);
            if (ov[k] >= LIM || ov[k] <= -LIM) reporta(E_ACUM, kid, x + k, ov[k], -3);
        }
        grava_bloco4<false>(ov, ev - 8, (int8_t*)Oacc_, (int8_t*)Oe_, x, (size_t)(b0 + 16 * qt + r) * (D / 32) + (h * HD + c) / 32, kid);
        return;
    }
    int* Oacc = (int*)Oacc_;
    int16_t* Oe = (int16_t*)Oe_;
    // wave wv writes the 16 dimensions 16 wv .. 16 wv + 15
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int r = 4 * lg + v, c = 16 * wv + lr;
        const int ov = (int)(so[0][r][c] + so[1][r][c] + so[2][r][c] + so[3][r][c]);
        const size_t x = (size_t)(b0 + i0 + v) * D + h * HD + c;
        if (ov >= LIM || ov <= -LIM) reporta(E_ACUM, kid, x, ov, -3);
        Oacc[x] = ov;
        Oe[x] = (int16_t)(ev - 8);
    }
}

// ---------------------------------------------------------------------------------------------- backward
// The arithmetic of k_atb_mf_linhas / _gq / _gkv / k_atb_exp, in launches that read converted operands from the
// workspace and split each 16-row tile's partner tiles over four waves:
//   (0) k_atb_prep: head maxima of dO, q, k, v; dO, v as m8 << L fragments; k, q, dO aligned as f16 [64][T];
//       for the bound variant (LIMITE), per 64 tokens max |dO| and max ||v||_1 (ops.py:231-235); or k_atb_prep_s,
//       the same for dO alone when the forward's conversion pass saved those of q, k, v (exact variant);
//   (1) k_atb1 (exact variant): per query tile, max |gP| over its causal pairs;
//   (2) k_atb2: s_i = rnd(sum_j P_ij rnd(gP_ij, sh), 8) per row, and per query tile the maxima that set dS's
//       shrink (max |P (gP' - s)|, or max P, max |gP'|, max |s| for LIMITE);
//   (3a) k_atbq: gq_i = sum_j dS_ij k_j and the exponents of the q columns;
//   (3b) k_atbkv: gk_j = sum_i dS_ij q_i, gv_j = sum_i P_ij dO_i and the exponents of the k and v columns.
// Partial maxima sit in per-tile slots (no atomics, no clearing); the consumers reduce over the slots. The four
// waves' partial sums are exact integers below 2^31 and are added in 32 bits through LDS.
namespace atw {
constexpr int SLOTS = 32;            // per head and kind: T / 16 <= 32 query tiles
struct WsB {
    int8_t *gm8, *gL, *vm8, *vL;     // dO, v: m8 [BH][T][64] (chunks as km8's), L [BH][T][2]
    _Float16 *kt, *qt, *gt;          // k, q, dO aligned: f16 [BH][64][T] in fragment order (grava_ft64)
    int* sl;                         // s_i [BH][T]
    int* mx;                         // [BH][4]: ego, eq, ek, ev (head maxima - GA)
    int* p1a;                        // [BH][SLOTS]: max |gP| per query tile, or max |dO| per 64 tokens (LIMITE)
    int* p1b;                        // [BH][SLOTS]: max ||v||_1 per 64 tokens (LIMITE)
    int *p2a, *p2b, *p2c;            // [BH][SLOTS]: max |P (gP' - s)|, or max P, max |gP'|, max |s| (LIMITE)
    int* ds;                         // [BH][T/16 query tiles][T/16 key tiles][16][16]: P (gP' - s) before dS's shrink
};
// element (i, j) of head bh's dS before its shrink (|value| < 2^25: P <= 255, |gP' - s| < 2^17), in tile (i/16, j/16)
// at row i % 16, column j % 16; written by k_atb2 for the causal tiles, read by k_atbqkv
__device__ __forceinline__ size_t ds_pos(int bh, int nqt, int qt, int kt) { return (((size_t)bh * nqt + qt) * nqt + kt) * 256; }
inline size_t bytes_back(long long BH, int T) {
    const size_t n = (size_t)BH * T;
    return 2 * (alinha256(n * 64) + alinha256(n * 2)) + 3 * alinha256(n * 64 * 2) + alinha256(n * 4) + alinha256((size_t)BH * 16) +
           5 * alinha256((size_t)BH * SLOTS * 4) + alinha256((size_t)BH * T * T * 4);
}
inline WsB parte_b(void* base, long long BH, int T) {
    const size_t n = (size_t)BH * T;
    char* p = (char*)base;
    WsB w;
    w.gm8 = (int8_t*)p; p += alinha256(n * 64);
    w.gL = (int8_t*)p; p += alinha256(n * 2);
    w.vm8 = (int8_t*)p; p += alinha256(n * 64);
    w.vL = (int8_t*)p; p += alinha256(n * 2);
    w.kt = (_Float16*)p; p += alinha256(n * 64 * 2);
    w.qt = (_Float16*)p; p += alinha256(n * 64 * 2);
    w.gt = (_Float16*)p; p += alinha256(n * 64 * 2);
    w.sl = (int*)p; p += alinha256(n * 4);
    w.mx = (int*)p; p += alinha256((size_t)BH * 16);
    w.p1a = (int*)p; p += alinha256((size_t)BH * SLOTS * 4);
    w.p1b = (int*)p; p += alinha256((size_t)BH * SLOTS * 4);
    w.p2a = (int*)p; p += alinha256((size_t)BH * SLOTS * 4);
    w.p2b = (int*)p; p += alinha256((size_t)BH * SLOTS * 4);
    w.p2c = (int*)p; p += alinha256((size_t)BH * SLOTS * 4);
    w.ds = (int*)p;
    return w;
}
// maximum over the first n slots of head bh (every slot value is >= 0): lane i reads slot i (one load for the wave,
// not a chain of n dependent ones), then a wave-wide maximum; call from uniform control flow
__device__ __forceinline__ int max_slots(const int* s, int bh, int n) {
    const int lane = threadIdx.x & 63;
    const int x = s[(size_t)bh * SLOTS + min(lane, SLOTS - 1)];      // every lane loads (no branch): lanes past n
    return g_max<64>(lane < n ? x : 0);                               // count 0
}
template <int LIMITE>
__device__ __forceinline__ int sh_gp_ws(const WsB& w, int bh, int T) {
    if (LIMITE) return max(bitlen(max_slots(w.p1a, bh, T / 64) * max_slots(w.p1b, bh, T / 64)) - 15, 0);
    return max(bitlen(max_slots(w.p1a, bh, T / 16)) - 15, 0);
}
template <int LIMITE>
__device__ __forceinline__ int sh_ds_ws(const WsB& w, int bh, int T, int dsb) {
    const int n = T / 16;
    if (LIMITE) return max(bitlen(max_slots(w.p2a, bh, n) * (max_slots(w.p2b, bh, n) + max_slots(w.p2c, bh, n))) - dsb, 0);
    return max(bitlen(max_slots(w.p2a, bh, n)) - dsb, 0);
}
}

// workgroup maximum of a non-negative value (256 threads); red[4]
__device__ __forceinline__ int wg_max4(int v, int (&red)[4]) {
    v = g_max<64>(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const int r = max(max(red[0], red[1]), max(red[2], red[3]));
    __syncthreads();
    return r;
}

// GP (exact variant, T <= 256): the launch also computes max |gP| over the causal pairs of every query tile, what
// k_atb1 computes, into the same slots, in workgroups of their own that run beside the conversion workgroups:
// blocks [0, BH T/64) take the per-tile maxima, the next BH T/64 the conversions. Workgroup g of head bh takes
// query tiles {a, n - 1 - a} for a = g and a = n/2 - 1 - g (n = T/16 query tiles): 2 (n + 1) causal tile pairs,
// the same for every g, dealt round-robin to its four waves. It converts the dO rows of its four query tiles and v
// of keys 0 .. 16 (n - 1 - g) + 15 itself (m8 << L fragments in LDS, rows 72 bytes apart), so it waits for no
// other workgroup.
template <int LIMITE>
__device__ __forceinline__ void atb_gp(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE, const int8_t* __restrict__ qm,
                                       const int8_t* __restrict__ qE, atw::WsB& w, int T, int H, int D, int blk, int GA, int BH,
                                       int8_t* lds, int (&red)[4][4]) {
    constexpr int HD = 64, RS = 72;
    static_assert(3 * sizeof(TileT) >= 256 * RS + 64 * RS + 128 + 512, "atb_gp's LDS fits k_atb_prep's tiles");
    const int bh = (int)blockIdx.x % BH, g = (int)blockIdx.x / BH, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, tid = threadIdx.x, nbl = ld / blk, nbg = D / blk, nqt = T / 16;
    const int c4 = tid & 3, half = c4 >> 1, tl = tid >> 2, colg = h * HD + 16 * c4;
    const int a1 = g, a2 = nqt / 2 - 1 - g;
    const int qs0 = a1, qs1 = nqt - 1 - a1, qs2 = a2, qs3 = nqt - 1 - a2;
    const int nk = 16 * qs1 + 16;                                     // keys 0 .. nk - 1 (qs1 is the last tile)
    int8_t* vm_s = lds;                                               // [T][RS]
    int8_t* dm_s = vm_s + 256 * RS;                                   // [64][RS]: rows 16 i + r of query tile qs_i
    int8_t* dl_s = dm_s + 64 * RS;                                    // [64][2]
    int8_t* vl_s = dl_s + 128;                                        // [T][2]
    // every operand load first: v of 64-key chunk r (key 64 r + tl), dO of row tl of the four query tiles
    int4 rx[4];
    int ex[4];
#pragma unroll
    for (int r = 0; r < 4; r++)
        if (64 * r < nk) {
            const int key = 64 * r + tl;
            rx[r] = ld16(qm + (size_t)(b0 + key) * ld + 2 * D + colg);
            ex[r] = qE[(size_t)(b0 + key) * nbl + (2 * D + colg) / blk];
        }
    const int qti = tl >> 4, qt_l = qti == 0 ? qs0 : qti == 1 ? qs1 : qti == 2 ? qs2 : qs3;
    const int tq = 16 * qt_l + (tl & 15);
    const int4 rg = ld16(gom + (size_t)(b0 + tq) * D + colg);
    const int egt = goE[(size_t)(b0 + tq) * nbg + colg / blk];
    int emv, emg;
    {
        int mv = SEM_TOPO, mg = SEM_TOPO;
        for (int tk = tid; tk < T; tk += 256) {
            mv = max(mv, emx_fatia(qE + (size_t)(b0 + tk) * nbl, 2 * D + h * HD, blk));
            mg = max(mg, emx_fatia(goE + (size_t)(b0 + tk) * nbg, h * HD, blk));
        }
        mv = g_max<64>(mv);
        mg = g_max<64>(mg);
        if ((tid & 63) == 0) { red[0][tid >> 6] = mv; red[1][tid >> 6] = mg; }
        __syncthreads();
        emv = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
        emg = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));
    }
    auto guarda16 = [](int8_t* d, const int8_t (&m)[16]) {             // two 8-byte stores (rows are 8-byte aligned)
        long x = 0, y = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) { x |= (long)(uint8_t)m[k] << (8 * k); y |= (long)(uint8_t)m[8 + k] << (8 * k); }
        reinterpret_cast<long*>(d)[0] = x;
        reinterpret_cast<long*>(d)[1] = y;
    };
#pragma unroll
    for (int r = 0; r < 4; r++)
        if (64 * r < nk) {
            int v[16];
            abre_i8(rx[r], v);
            const int sft = emv - ex[r];
            int8_t m8[16];
            int L = 0;
#pragma unroll
            for (int k = 0; k < 16; k++) { int x; m8_L(v[k], sft, GA, x, L); m8[k] = (int8_t)x; }
            guarda16(vm_s + (64 * r + tl) * RS + 16 * c4, m8);
            if ((c4 & 1) == 0) vl_s[(64 * r + tl) * 2 + half] = (int8_t)L;
        }
    {
        int v[16];
        abre_i8(rg, v);
        const int sft = emg - egt;
        int8_t m8[16];
        int L = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) { int x; m8_L(v[k], sft, GA, x, L); m8[k] = (int8_t)x; }
        guarda16(dm_s + tl * RS + 16 * c4, m8);
        if ((c4 & 1) == 0) dl_s[tl * 2 + half] = (int8_t)L;
    }
    __syncthreads();
    // pair k of the list (query tile i, key tile kt) for kt = 0 .. qs_i, i = 0 .. 3, goes to wave k % 4
    const int wv = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
    const int n0 = qs0 + 1, n01 = n0 + qs1 + 1, n012 = n01 + qs2 + 1, np = n012 + qs3 + 1;
    int mg0 = 0, mg1 = 0, mg2 = 0, mg3 = 0;
    for (int k0 = wv; k0 < np; k0 += 16) {                             // four pairs in flight
        long da0[4], da1[4], vb0[4], vb1[4];
        int lxs[4][2], l0[4], l1[4], iq[4], ktile[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int k = min(k0 + 4 * u, np - 1);                    // past the list: a repeat, not counted
            const int i = k < n0 ? 0 : k < n01 ? 1 : k < n012 ? 2 : 3;
            const int kt = k - (i == 0 ? 0 : i == 1 ? n0 : i == 2 ? n01 : n012);
            iq[u] = i; ktile[u] = kt;
            const int8_t* da = dm_s + (16 * i + lr) * RS + 8 * lg;
            da0[u] = *reinterpret_cast<const long*>(da);
            da1[u] = *reinterpret_cast<const long*>(da + 32);
            const long lxw = *reinterpret_cast<const long*>(dl_s + (16 * i + 4 * lg) * 2);   // L of rows 4 lg .. 4 lg + 3
            lxs[u][0] = (int)lxw; lxs[u][1] = (int)(lxw >> 32);
            const int j = 16 * kt + lr;
            const int8_t* vb = vm_s + j * RS + 8 * lg;
            vb0[u] = *reinterpret_cast<const long*>(vb);
            vb1[u] = *reinterpret_cast<const long*>(vb + 32);
            const int lv = *reinterpret_cast<const unsigned short*>(vl_s + j * 2);
            l0[u] = (int)(int8_t)lv; l1[u] = (int)(int8_t)(lv >> 8);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (k0 + 4 * u >= np) break;                               // uniform
            const int i = iq[u], qt = i == 0 ? qs0 : i == 1 ? qs1 : i == 2 ? qs2 : qs3;
            int lx[4][2];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int wd = lxs[u][v >> 1] >> (16 * (v & 1));
                lx[v][0] = (int)(int8_t)wd; lx[v][1] = (int)(int8_t)(wd >> 8);
            }
            int o[4];
            tile_xyt(da0[u], da1[u], vb0[u], vb1[u], lx, l0[u], l1[u], o);
            const int j = 16 * ktile[u] + lr, i0 = 16 * qt + 4 * lg;
            int m = 0;
#pragma unroll
            for (int v = 0; v < 4; v++) if (j <= i0 + v) m = max(m, abs(o[v]));
            mg0 = i == 0 ? max(mg0, m) : mg0;
            mg1 = i == 1 ? max(mg1, m) : mg1;
            mg2 = i == 2 ? max(mg2, m) : mg2;
            mg3 = i == 3 ? max(mg3, m) : mg3;
        }
    }
    mg0 = g_max<64>(mg0); mg1 = g_max<64>(mg1); mg2 = g_max<64>(mg2); mg3 = g_max<64>(mg3);
    __syncthreads();                                                   // red was read above by every thread
    if (lane == 0) { red[wv][0] = mg0; red[wv][1] = mg1; red[wv][2] = mg2; red[wv][3] = mg3; }
    __syncthreads();
    if (tid < 4) {
        const int qt = tid == 0 ? qs0 : tid == 1 ? qs1 : tid == 2 ? qs2 : qs3;
        w.p1a[bh * atw::SLOTS + qt] = max(max(red[0][tid], red[1][tid]), max(red[2][tid], red[3][tid]));
    }
}

template <int LIMITE, bool GP = false>
__global__ void __launch_bounds__(256) k_atb_prep(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE, const int8_t* __restrict__ qm,
                                                  const int8_t* __restrict__ qE, atw::WsB w, int T, int H, int D, int blk, int GA) {
    constexpr int HD = 64;
    __shared__ int red[4][4];
    __shared__ int red1[4];
    __shared__ __align__(16) TileT tiles[3];                         // dO, q, k; or atb_gp's fragments (23.7 KB)
    TileT &tg = tiles[0], &tq = tiles[1], &tk = tiles[2];
    const int nparts = T / 64;
    int wg = (int)blockIdx.x;
    if constexpr (GP) {
        static_assert(LIMITE == 0, "per-tile max |gP| belongs to the exact variant");
        const int BH = (int)gridDim.x / (2 * nparts);
        if (wg < BH * nparts) {                                        // uniform per workgroup
            atb_gp<LIMITE>(gom, goE, qm, qE, w, T, H, D, blk, GA, BH, reinterpret_cast<int8_t*>(&tiles[0][0][0]), red);
            return;
        }
        wg -= BH * nparts;
    }
    const int bh = wg / nparts, part = wg % nparts, b = bh / H, h = bh % H;
    const int ld = 3 * D, b0 = b * T, tid = threadIdx.x, nbl = ld / blk, nbg = D / blk;
    // thread (t, c4): dimensions 16 c4 .. 16 c4 + 15 of token t. Every value it converts is loaded first, so the
    // loads overlap the head maxima's reduction below.
    const int t = part * 64 + (tid >> 2), c4 = tid & 3, half = c4 >> 1;
    const size_t tt = (size_t)bh * T + t, lq = (size_t)(b0 + t) * ld;
    const int colg = h * HD + 16 * c4;
    const int4 rg = ld16(gom + (size_t)(b0 + t) * D + colg), rv = ld16(qm + lq + 2 * D + colg);
    const int4 rq = ld16(qm + lq + colg), rk = ld16(qm + lq + D + colg);
    const int egt = goE[(size_t)(b0 + t) * nbg + colg / blk], evt = qE[(size_t)(b0 + t) * nbl + (2 * D + colg) / blk];
    const int eqt = qE[(size_t)(b0 + t) * nbl + colg / blk], ekt = qE[(size_t)(b0 + t) * nbl + (D + colg) / blk];
    // head maxima of the q, k, v and dO exponents in one reduction
    int emq, emk, emv, emg;
    {
        int m[4] = {SEM_TOPO, SEM_TOPO, SEM_TOPO, SEM_TOPO};
        for (int tk = tid; tk < T; tk += 256) {                      // one token per thread (T <= 512: at most two)
            const int8_t* e = qE + (size_t)(b0 + tk) * nbl;
            m[0] = max(m[0], emx_fatia(e, h * HD, blk));
            m[1] = max(m[1], emx_fatia(e, D + h * HD, blk));
            m[2] = max(m[2], emx_fatia(e, 2 * D + h * HD, blk));
            m[3] = max(m[3], emx_fatia(goE + (size_t)(b0 + tk) * nbg, h * HD, blk));
        }
#pragma unroll
        for (int x = 0; x < 4; x++) m[x] = g_max<64>(m[x]);
        if ((tid & 63) == 0)
#pragma unroll
            for (int x = 0; x < 4; x++) red[x][tid >> 6] = m[x];
        __syncthreads();
        emq = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
        emk = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));
        emv = max(max(red[2][0], red[2][1]), max(red[2][2], red[2][3]));
        emg = max(max(red[3][0], red[3][1]), max(red[3][2], red[3][3]));
    }
    if (part == 0 && tid == 0) { w.mx[bh * 4] = emg - GA; w.mx[bh * 4 + 1] = emq - GA; w.mx[bh * 4 + 2] = emk - GA; w.mx[bh * 4 + 3] = emv - GA; }
    int amax = 0, v1 = 0;
    {   // dO: m8 << L fragments and aligned f16
        int v[16];
        abre_i8(rg, v);
        const int s = emg - egt;
        const Desl ds(s);
        int8_t m8[16];
        int L = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            int a; m8_L(v[k], s, GA, a, L); m8[k] = (int8_t)a;
            const int al = ds(shl(v[k], GA));
            amax = max(amax, abs(al));
            tg[16 * c4 + k][tid >> 2] = (_Float16)al;
        }
        grava_m8_fragmentos(w.gm8 + tt * 64, c4, m8);
        if ((c4 & 1) == 0) w.gL[tt * 2 + half] = (int8_t)L;
    }
    {   // v: m8 << L fragments (and ||v||_1 for LIMITE)
        int v[16];
        abre_i8(rv, v);
        const int s = emv - evt;
        const Desl ds(s);
        int8_t m8[16];
        int L = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            int a; m8_L(v[k], s, GA, a, L); m8[k] = (int8_t)a;
            if (LIMITE) v1 += abs(ds(shl(v[k], GA)));
        }
        grava_m8_fragmentos(w.vm8 + tt * 64, c4, m8);
        if ((c4 & 1) == 0) w.vL[tt * 2 + half] = (int8_t)L;
    }
#pragma unroll
    for (int x = 0; x < 2; x++) {   // q (x = 0), k (x = 1): aligned f16, transposed
        int v[16];
        abre_i8(x ? rk : rq, v);
        const Desl ds((x ? emk : emq) - (x ? ekt : eqt));
        TileT& dst = x ? tk : tq;
#pragma unroll
        for (int k = 0; k < 16; k++) dst[16 * c4 + k][tid >> 2] = (_Float16)ds(shl(v[k], GA));
    }
    __syncthreads();
    grava_ft64(tg, w.gt + (size_t)bh * 64 * T, part * 64);
    grava_ft64(tq, w.qt + (size_t)bh * 64 * T, part * 64);
    grava_ft64(tk, w.kt + (size_t)bh * 64 * T, part * 64);
    if (LIMITE) {
        v1 = quad_soma(v1);
        const int a = wg_max4(amax, red1), c = wg_max4(v1, red1);
        if (tid == 0) { w.p1a[bh * atw::SLOTS + part] = a; w.p1b[bh * atw::SLOTS + part] = c; }
    }
}

// k_atb_prep of the exact variant when the forward's conversion pass saved q, k, v (atw::Salvo, the same qkv): the
// workspace's vm8, vL, kt, qt point into the saved buffer, so only dO is converted here; the head maxima of q, k, v
// come from the saved ones (smx), that of dO from one reduction.
__global__ void __launch_bounds__(256) k_atb_prep_s(const int8_t* __restrict__ gom, const int8_t* __restrict__ goE, atw::WsB w,
                                                    const int* __restrict__ smx, int T, int H, int D, int blk, int GA) {
    constexpr int HD = 64;
    __shared__ int red[4];
    __shared__ __align__(16) TileT tg;
    const int nparts = T / 64, bh = blockIdx.x / nparts, part = blockIdx.x % nparts, b = bh / H, h = bh % H;
    const int b0 = b * T, tid = threadIdx.x, nbg = D / blk;
    const int t = part * 64 + (tid >> 2), c4 = tid & 3, half = c4 >> 1;
    const size_t tt = (size_t)bh * T + t;
    const int colg = h * HD + 16 * c4;
    const int4 rg = ld16(gom + (size_t)(b0 + t) * D + colg);
    const int egt = goE[(size_t)(b0 + t) * nbg + colg / blk];
    int m = SEM_TOPO;
    for (int tk = tid; tk < T; tk += 256) m = max(m, emx_fatia(goE + (size_t)(b0 + tk) * nbg, h * HD, blk));   // T <= 512
    m = g_max<64>(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const int emg = max(max(red[0], red[1]), max(red[2], red[3]));
    if (part == 0 && tid == 0) {
        w.mx[bh * 4] = emg - GA;
        w.mx[bh * 4 + 1] = smx[bh * 4] - GA; w.mx[bh * 4 + 2] = smx[bh * 4 + 1] - GA; w.mx[bh * 4 + 3] = smx[bh * 4 + 2] - GA;
    }
    {   // dO: m8 << L fragments and aligned f16, as k_atb_prep
        int v[16];
        abre_i8(rg, v);
        const int s = emg - egt;
        const Desl ds(s);
        int8_t m8[16];
        int L = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            int a; m8_L(v[k], s, GA, a, L); m8[k] = (int8_t)a;
            tg[16 * c4 + k][tid >> 2] = (_Float16)ds(shl(v[k], GA));
        }
        grava_m8_fragmentos(w.gm8 + tt * 64, c4, m8);
        if ((c4 & 1) == 0) w.gL[tt * 2 + half] = (int8_t)L;
    }
    __syncthreads();
    grava_ft64(tg, w.gt + (size_t)bh * 64 * T, part * 64);
}

// gP tile of query rows i0 .. i0 + 3 (this lane) x key j = 16 t + lr from the workspace fragments
struct FragQ {                                      // dO fragments of a query tile (A operand) and their L
    long ga[2];
    int lx[4][2];
};
__device__ __forceinline__ FragQ frag_q(const atw::WsB& w, size_t hb, int qt, int lr, int lg) {
    FragQ f;
    const size_t ia = hb + 16 * qt + lr, i0 = hb + 16 * qt + 4 * lg;
    le_m8_fragmentos(w.gm8 + ia * 64, lg, f.ga[0], f.ga[1]);
#pragma unroll
    for (int v = 0; v < 4; v++) { f.lx[v][0] = w.gL[(i0 + v) * 2]; f.lx[v][1] = w.gL[(i0 + v) * 2 + 1]; }
    return f;
}
__device__ __forceinline__ void gp_tile(const atw::WsB& w, size_t hb, const FragQ& f, int t, int lr, int lg, int (&o)[4]) {
    const size_t j = hb + 16 * t + lr;
    long v0, v1;
    le_m8_fragmentos(w.vm8 + j * 64, lg, v0, v1);
    tile_xyt(f.ga[0], f.ga[1], v0, v1, f.lx, w.vL[j * 2], w.vL[j * 2 + 1], o);
}
// query tile of this workgroup, in decreasing work across all heads (tile qt pairs with qt + 1 key tiles)
#define ATB_TILE_Q ATB_TILE_Q_(blockIdx.x, gridDim.x)
#define ATB_TILE_Q_(BX, GX)                                                                                            \
    const int nqt = T / 16, BH = (GX) / nqt, bh = (BX) % BH, qt = nqt - 1 - (int)((BX) / BH);                          \
    const int b = bh / H, h = bh % H, b0 = b * T;                                                                      \
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lr = lane & 15, lg = lane >> 4; \
    const size_t hb = (size_t)bh * T;                                                                                  \
    const int i0 = 16 * qt + 4 * lg, nv = qt >= wv ? (qt - wv) / 4 + 1 : 0;

template <int NTW>
__global__ void __launch_bounds__(256) k_atb1(atw::WsB w, int T, int H) {
    __shared__ int red[4];
    ATB_TILE_Q
    (void)b0;
    const FragQ f = frag_q(w, hb, qt, lr, lg);
    int mg = 0;
#pragma unroll
    for (int n = 0; n < NTW; n++) {
        if (n >= nv) continue;
        const int t = wv + 4 * n, j = 16 * t + lr;
        int o[4];
        gp_tile(w, hb, f, t, lr, lg, o);
#pragma unroll
        for (int v = 0; v < 4; v++) if (j <= i0 + v) mg = max(mg, abs(o[v]));
    }
    mg = wg_max4(mg, red);
    if (tid == 0) w.p1a[bh * atw::SLOTS + qt] = mg;
}

template <int NTW, int LIMITE>
__global__ void __launch_bounds__(256) k_atb2(atw::WsB w, const uint8_t* __restrict__ P, int T, int H, int D, int kid) {
    __shared__ int red[4];
    __shared__ int sred[4][16];
    ATB_TILE_Q
    const FragQ f = frag_q(w, hb, qt, lr, lg);
    const int sh = atw::sh_gp_ws<LIMITE>(w, bh, T);                  // after frag_q's loads are issued
    const Desl dsh(sh);                                              // gP's shrink, one shift per head
    const uint8_t* Pb = P + (size_t)bh * T * T;
    int x[NTW][4];
    unsigned pr[NTW];
    int s[4] = {0, 0, 0, 0}, pm = 0, gm = 0;
#pragma unroll
    for (int n = 0; n < NTW; n++) {
        if (n >= nv) continue;
        const int t = wv + 4 * n, j = 16 * t + lr;
        int o[4];
        gp_tile(w, hb, f, t, lr, lg, o);
        pr[n] = *reinterpret_cast<const unsigned*>(Pb + (size_t)j * T + i0);     // P_ij, rows i0 .. i0 + 3
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int xv = j <= i0 + v ? dsh(o[v]) : 0;
            const int p = (pr[n] >> (8 * v)) & 255;
            x[n][v] = xv;
            s[v] += mul24(p, xv);
            if (LIMITE) { pm = max(pm, p); gm = max(gm, abs(xv)); }
        }
    }
#pragma unroll
    for (int v = 0; v < 4; v++) s[v] = g_sum<16>(s[v]);
    if (lr == 0)
#pragma unroll
        for (int v = 0; v < 4; v++) sred[wv][4 * lg + v] = s[v];
    __syncthreads();
    const int ld = 3 * D;
    int sl[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int tot = sred[0][4 * lg + v] + sred[1][4 * lg + v] + sred[2][4 * lg + v] + sred[3][4 * lg + v];
        if ((tot >= LIM || tot <= -LIM) && lr == 0 && wv == 0) reporta(E_ACUM, kid, (long long)(b0 + i0 + v) * ld + h * 64, tot, -4);
        sl[v] = rnd_d(tot, 8);
        if (lr == 0 && wv == 0) w.sl[hb + i0 + v] = sl[v];
    }
    // dS before its shrink, P (gP' - s) (0 past the diagonal, where P = 0), for k_atbqkv: rows 4 lg + v of tile
    // (qt, t), column lr
    int md = 0;
#pragma unroll
    for (int n = 0; n < NTW; n++) {
        if (n >= nv) continue;
        int* dt = w.ds + atw::ds_pos(bh, nqt, qt, wv + 4 * n) + 16 * 4 * lg + lr;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int d = mul24((int)((pr[n] >> (8 * v)) & 255), x[n][v] - sl[v]);
            dt[16 * v] = d;
            md = max(md, abs(d));
        }
    }
    if (LIMITE) {
        const int a = wg_max4(pm, red), c = wg_max4(gm, red);
        const int d = wg_max4(max(max(abs(sl[0]), abs(sl[1])), max(abs(sl[2]), abs(sl[3]))), red);
        if (tid == 0) { w.p2a[bh * atw::SLOTS + qt] = a; w.p2b[bh * atw::SLOTS + qt] = c; w.p2c[bh * atw::SLOTS + qt] = d; }
    } else {
        md = wg_max4(md, red);
        if (tid == 0) w.p2a[bh * atw::SLOTS + qt] = md;
    }
}

// sums the four waves' partials parc[w][16][64] (this lane: rows 4 lg + v, column 16 dt + lr of wave wv's
// registers) -- written by every wave, then wave wv adds column group 16 wv .. 16 wv + 15 -- into out[v]. The sums
// are the exact integer results of at most 256 products |dS| |k| <= 4096 * 2032 (or P |dO| <= 255 * 2032), below
// 2^31: 32-bit adds (modular, unsigned) give them exactly, as the int64 sums of the arithmetic would.
__device__ __forceinline__ void soma_ondas(int (&parc)[4][16][64], const int (&mine)[4][4], int wv, int lr, int lg, int (&out)[4]) {
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) parc[wv][4 * lg + v][16 * dt + lr] = mine[dt][v];
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int r = 4 * lg + v, c = 16 * wv + lr;
        out[v] = (int)((unsigned)parc[0][r][c] + (unsigned)parc[1][r][c] + (unsigned)parc[2][r][c] + (unsigned)parc[3][r][c]);
    }
    __syncthreads();
}

// as soma_ondas, read back in the block layout of grava_bloco4: out[k] = row tid / 16, column 4 (tid % 16) + k
__device__ __forceinline__ void soma_ondas_bloco(int (&parc)[4][16][64], const int (&mine)[4][4], int wv, int lr, int lg, int (&out)[4]) {
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) parc[wv][4 * lg + v][16 * dt + lr] = mine[dt][v];
    __syncthreads();
    const int r = threadIdx.x >> 4, c = 4 * (threadIdx.x & 15);
#pragma unroll
    for (int k = 0; k < 4; k++)
        out[k] = (int)((unsigned)parc[0][r][c + k] + (unsigned)parc[1][r][c + k] + (unsigned)parc[2][r][c + k] + (unsigned)parc[3][r][c + k]);
    __syncthreads();
}

// gq of workgroup blk of nblk. lds: dS tiles, then (after a barrier) the waves' 32-bit partial sums in the same
// LDS (LDS_ATBQKV bytes).
template <int NTW, int LIMITE, bool BLOCO = false>
__device__ __forceinline__ void atbq_corpo(const atw::WsB& w, const uint8_t* __restrict__ P, int* __restrict__ Gacc, int16_t* __restrict__ Ge,
                                           int T, int H, int D, int dsb, int kid, char* lds, const int blk, const int nblk) {
    constexpr int LP = 16 * (NTW + 1);
    auto dw = reinterpret_cast<short (*)[16][LP]>(lds);
    auto& parc = *reinterpret_cast<int (*)[4][16][64]>(lds);
    ATB_TILE_Q_(blk, nblk)
    (void)P;
    // dS before its shrink, as k_atb2 stored it (0 past the diagonal): rows 4 lg + v of tile (qt, t), column lr
    int dr[NTW][4];
#pragma unroll
    for (int n = 0; n < NTW; n++) {                                  // loads of every n issued together: tiles past
        const int t = min(wv + 4 * n, qt);                           // this wave's last re-read tile qt, unused
        const int* dt = w.ds + atw::ds_pos(bh, nqt, qt, t) + 16 * 4 * lg + lr;
#pragma unroll
        for (int v = 0; v < 4; v++) dr[n][v] = dt[16 * v];
    }
    // the head maxima after the loads above are issued (their slot reads need a reduction before any use)
    const int sh = atw::sh_gp_ws<LIMITE>(w, bh, T), sh2 = atw::sh_ds_ws<LIMITE>(w, bh, T, dsb);
    const Desl dsh2(sh2);                                            // dS's shrink, one shift per head
    const int ego = w.mx[bh * 4], ek = w.mx[bh * 4 + 2], ev = w.mx[bh * 4 + 3];
    const int eds = ego + ev + sh - 9 + sh2;
#pragma unroll
    for (int n = 0; n < NTW; n++) {
        if (n >= nv) continue;
#pragma unroll
        for (int v = 0; v < 4; v++) dw[wv][4 * lg + v][16 * n + lr] = (short)dsh2(dr[n][v]);
    }
    if (nv & 1)
#pragma unroll
        for (int v = 0; v < 4; v++) dw[wv][4 * lg + v][16 * nv + lr] = 0;
    __syncthreads();
    // gq partial = dS K over this wave's key tiles, in pairs; dS = a 256 + b 16 + c (see the MFMA backward above)
    f4_t acc[4][3] = {};
#pragma unroll
    for (int m = 0; m < (NTW + 1) / 2; m++) {
        if (2 * m >= nv) continue;
        h8_t pa, pb, pc;
        pedacos_ds(*reinterpret_cast<const s8_t*>(&dw[wv][lr][32 * m + 8 * lg]), pa, pb, pc);
        int tk = wv + 4 * (2 * m + (lg >> 1));
        if (tk >= nqt) tk = wv;                                      // pad tile: dS = 0 there
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            const h8_t kv = *reinterpret_cast<const h8_t*>(w.kt + (size_t)bh * 64 * T + pos_ft(tk, dt, lg & 1, lr));
            acc[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, kv, acc[dt][0], 0, 0, 0);
            acc[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pb, kv, acc[dt][1], 0, 0, 0);
            acc[dt][2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pc, kv, acc[dt][2], 0, 0, 0);
        }
    }
    int mine[4][4], gq[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) mine[dt][v] = junta3(acc[dt][0][v], acc[dt][1][v], acc[dt][2][v]);
    const int ld = 3 * D;
    __syncthreads();                                                 // every wave is done with dw: parc reuses it
    if constexpr (BLOCO) {                                           // Gacc, Ge: int8 mantissas and exponents
        soma_ondas_bloco(parc, mine, wv, lr, lg, gq);
        const int r = tid >> 4, c = 4 * (tid & 15);
        const size_t x = (size_t)(b0 + 16 * qt + r) * ld + h * 64 + c;
        int g4[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (gq[k] >= LIM || gq[k] <= -LIM) reporta(E_ACUM, kid, x + k, gq[k], -5);
            g4[k] = (int)gq[k];
        }
        grava_bloco4(g4, eds + ek, (int8_t*)Gacc, (int8_t*)Ge, x, (size_t)(b0 + 16 * qt + r) * (ld / 32) + (h * 64 + c) / 32, kid);
        return;
    }
    soma_ondas(parc, mine, wv, lr, lg, gq);
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const size_t o = (size_t)(b0 + i0 + v) * ld + h * 64 + 16 * wv + lr;
        if (gq[v] >= LIM || gq[v] <= -LIM) reporta(E_ACUM, kid, o, gq[v], -5);
        Gacc[o] = (int)gq[v];
        Ge[o] = (int16_t)(eds + ek);
    }
}

// gk, gv of workgroup blk of nblk. lds: dS and P tiles, then (after a barrier) the waves' 32-bit partial sums in
// the same LDS (LDS_ATBQKV bytes).
template <int NTW> constexpr size_t LDS_ATBQKV = cmax_(sizeof(short) * 4 * 16 * 16 * (NTW + 1) + 4 * 16 * 16 * (NTW + 1), sizeof(int) * 4 * 16 * 64);
template <int NTW, int LIMITE, bool BLOCO = false>
__device__ __forceinline__ void atbkv_corpo(const atw::WsB& w, const uint8_t* __restrict__ P, int* __restrict__ Gacc, int16_t* __restrict__ Ge,
                                            int T, int H, int D, int dsb, int kid, char* lds, const int blk, const int nblk) {
    constexpr int LP = 16 * (NTW + 1);
    auto dw = reinterpret_cast<short (*)[16][LP]>(lds);
    auto pw = reinterpret_cast<uint8_t (*)[16][LP]>(lds + sizeof(short) * 4 * 16 * LP);
    auto& parc = *reinterpret_cast<int (*)[4][16][64]>(lds);
    // key tile kt pairs with the query tiles kt .. nqt - 1: decreasing work is increasing kt
    const int nqt = T / 16, BH = nblk / nqt, bh = blk % BH, kt = (int)(blk / BH);
    const int b = bh / H, h = bh % H, b0 = b * T;
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lr = lane & 15, lg = lane >> 4;
    const size_t hb = (size_t)bh * T;
    const int nv = (nqt - kt - wv + 3) / 4;                          // this wave's query tiles kt + wv + 4 n, n < nv
    const int jr = 16 * kt + 4 * lg;                                 // this lane's 4 keys jr .. jr + 3
    const uint8_t* Pb = P + (size_t)bh * T * T;
    // dS before its shrink, as k_atb2 stored it (0 past the diagonal): row lr (query 16 t + lr) of tile (t, kt),
    // columns 4 lg .. 4 lg + 3 (this lane's keys), one 16-byte load; P of the same pairs
    int4 dr[NTW];
#pragma unroll
    for (int n = 0; n < NTW; n++) {                                  // loads of every n issued together: tiles past
        const int t = min(kt + wv + 4 * n, nqt - 1);                 // this wave's last re-read tile nqt - 1, unused
        dr[n] = *reinterpret_cast<const int4*>(w.ds + atw::ds_pos(bh, nqt, t, kt) + 16 * lr + 4 * lg);
    }
    // P of the tile's 16 keys against query tiles kt .. nqt - 1: 16 rows of the [j][i] storage, one 16-byte piece
    // (query tile kt + c, key 16 kt + r) per thread and column group, staged for the wave that owns query tile kt + c
    constexpr int NC = NTW / 4;
    const int r = tid >> 4;
    int4 pq[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {                                  // unconditional: past the last query tile it
        const int t = min(kt + (tid & 15) + 16 * c, nqt - 1);         // re-reads that tile, unused
        pq[c] = *reinterpret_cast<const int4*>(Pb + (size_t)(16 * kt + r) * T + 16 * t);
    }
    // the head maxima after the loads above are issued
    const int sh = atw::sh_gp_ws<LIMITE>(w, bh, T), sh2 = atw::sh_ds_ws<LIMITE>(w, bh, T, dsb);
    const Desl dsh2(sh2);                                            // dS's shrink, one shift per head
    const int ego = w.mx[bh * 4], eq = w.mx[bh * 4 + 1], ev = w.mx[bh * 4 + 3];
    const int eds = ego + ev + sh - 9 + sh2;
#pragma unroll
    for (int n = 0; n < NTW; n++) {
        if (n >= nv) continue;
        const int d4[4] = {dr[n].x, dr[n].y, dr[n].z, dr[n].w};
#pragma unroll
        for (int v = 0; v < 4; v++) dw[wv][4 * lg + v][16 * n + lr] = (short)dsh2(d4[v]);
    }
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int cc = (tid & 15) + 16 * c, t = kt + cc;
        if (t >= nqt) continue;
        int4 q = pq[c];
        if (t == kt) {                                               // the diagonal tile: P = 0 for queries before key r
            unsigned x[4] = {(unsigned)q.x, (unsigned)q.y, (unsigned)q.z, (unsigned)q.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int z = min(max(r - 4 * k, 0), 4);             // bytes of word k below the diagonal
                x[k] &= z == 4 ? 0u : (~0u << (8 * z));
            }
            q = make_int4((int)x[0], (int)x[1], (int)x[2], (int)x[3]);
        }
        *reinterpret_cast<int4*>(&pw[cc & 3][r][16 * (cc >> 2)]) = q;
    }
    if (nv & 1)
#pragma unroll
        for (int v = 0; v < 4; v++) { dw[wv][4 * lg + v][16 * nv + lr] = 0; pw[wv][4 * lg + v][16 * nv + lr] = 0; }
    __syncthreads();
    f4_t ak[4][3] = {}, av[4][2] = {};
#pragma unroll
    for (int m = 0; m < (NTW + 1) / 2; m++) {
        if (2 * m >= nv) continue;
        h8_t pa, pb, pc, ph, pl;
        pedacos_ds(*reinterpret_cast<const s8_t*>(&dw[wv][lr][32 * m + 8 * lg]), pa, pb, pc);
        const uint8_t* pp = &pw[wv][lr][32 * m + 8 * lg];
#pragma unroll
        for (int k = 0; k < 8; k++) { ph[k] = (_Float16)(pp[k] >> 4); pl[k] = (_Float16)(pp[k] & 15); }
        int tq = kt + wv + 4 * (2 * m + (lg >> 1));
        if (tq >= nqt) tq = kt + wv;                                 // pad tile: dS = P = 0 there
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            const size_t r = (size_t)bh * 64 * T + pos_ft(tq, dt, lg & 1, lr);
            const h8_t qv = *reinterpret_cast<const h8_t*>(w.qt + r);
            const h8_t gv = *reinterpret_cast<const h8_t*>(w.gt + r);
            ak[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, qv, ak[dt][0], 0, 0, 0);
            ak[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pb, qv, ak[dt][1], 0, 0, 0);
            ak[dt][2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pc, qv, ak[dt][2], 0, 0, 0);
            av[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, gv, av[dt][0], 0, 0, 0);
            av[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, gv, av[dt][1], 0, 0, 0);
        }
    }
    int mine[4][4], gk[4], gvv[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) mine[dt][v] = junta3(ak[dt][0][v], ak[dt][1][v], ak[dt][2][v]);
    const int ld = 3 * D;
    __syncthreads();                                                 // every wave is done with dw, pw: parc reuses them
    if constexpr (BLOCO) {                                           // Gacc, Ge: int8 mantissas and exponents
        soma_ondas_bloco(parc, mine, wv, lr, lg, gk);
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int v = 0; v < 4; v++) mine[dt][v] = junta2(av[dt][0][v], av[dt][1][v]);
        soma_ondas_bloco(parc, mine, wv, lr, lg, gvv);
        const int r = tid >> 4, c = 4 * (tid & 15);
        const size_t x = (size_t)(b0 + 16 * kt + r) * ld + h * 64 + c, xe = (size_t)(b0 + 16 * kt + r) * (ld / 32) + (h * 64 + c) / 32;
        int a4[4], b4[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (gk[k] >= LIM || gk[k] <= -LIM) reporta(E_ACUM, kid, x + D + k, gk[k], -5);
            if (gvv[k] >= LIM || gvv[k] <= -LIM) reporta(E_ACUM, kid, x + 2 * D + k, gvv[k], -5);
            a4[k] = (int)gk[k];
            b4[k] = (int)gvv[k];
        }
        grava_bloco4(a4, eds + eq, (int8_t*)Gacc, (int8_t*)Ge, x + D, xe + D / 32, kid);
        grava_bloco4(b4, ego - 8, (int8_t*)Gacc, (int8_t*)Ge, x + 2 * D, xe + 2 * D / 32, kid);
        return;
    }
    soma_ondas(parc, mine, wv, lr, lg, gk);
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) mine[dt][v] = junta2(av[dt][0][v], av[dt][1][v]);
    soma_ondas(parc, mine, wv, lr, lg, gvv);
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const size_t o = (size_t)(b0 + jr + v) * ld + h * 64 + 16 * wv + lr;
        if (gk[v] >= LIM || gk[v] <= -LIM) reporta(E_ACUM, kid, o + D, gk[v], -5);
        if (gvv[v] >= LIM || gvv[v] <= -LIM) reporta(E_ACUM, kid, o + 2 * D, gvv[v], -5);
        Gacc[o + D] = (int)gk[v];
        Gacc[o + 2 * D] = (int)gvv[v];
        Ge[o + D] = (int16_t)(eds + eq);
        Ge[o + 2 * D] = (int16_t)(ego - 8);
    }
}

// gk, gv (workgroups [0, G)) and gq (workgroups [G, 2G)) of the backward in one launch. Both read only what
// k_atb_prep and k_atb2 wrote and write disjoint columns of G, so their latency-bound workgroups run side by side
// (16 KiB of LDS and at most 64 VGPRs each: all 2G workgroups of config 4 are resident at once).
template <int NTW, int LIMITE, bool BLOCO = false>
__global__ void __launch_bounds__(256) k_atbqkv(atw::WsB w, const uint8_t* __restrict__ P, int* __restrict__ Gacc, int16_t* __restrict__ Ge,
                                                int T, int H, int D, int dsb, int kid) {
    __shared__ __align__(16) char lds[LDS_ATBQKV<NTW>];
    const int G = (int)gridDim.x / 2;
    if ((int)blockIdx.x < G) atbkv_corpo<NTW, LIMITE, BLOCO>(w, P, Gacc, Ge, T, H, D, dsb, kid, lds, (int)blockIdx.x, G);
    else atbq_corpo<NTW, LIMITE, BLOCO>(w, P, Gacc, Ge, T, H, D, dsb, kid, lds, (int)blockIdx.x - G, G);
}
