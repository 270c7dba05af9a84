// Block-exponent INT8 GEMM on CDNA4 i8 MFMA: C = A . B^T, A [M, K] and B [N, K] blocked along K.
//
// Arithmetic (ops.py:95-108): RA_i = max_b ea_ib, RB_j = max_b eb_jb; for every K-block b the exact product
// p_ijb = sum_{k in b} a_ik b_jk (one MFMA per 32 values of K), then acc_ij += rnd(p_ijb << 4, sa + sb) with
// sa = RA_i - ea_ib, sb = RB_j - eb_jb, round half to even; base_ij = RA_i + RB_j - 4.
//
// The rounding runs in fp64 with the round-to-nearest-even of the FMA itself:
//   g = fma(ldexp(double(p), 4 - sa), 2^-sb, 1.5 * 2^52).
// ldexp and the product by a power of two are exact, and |p * 2^(4 - sa - sb)| < 2^26 (|p| <= 128 * 128 * BLK),
// so the exact sum lies in [2^52, 2^53), where the spacing of doubles is 1: the FMA's one rounding is
// rnd(p << 4, sa + sb), and the low 32 bits of g are that integer in two's complement (1.5 * 2^52 has zero low
// bits). The row term is a 32-bit ldexp operand and the column term one double per column and block, so per
// output and K-block the work is cvt, ldexp, fma and add: 4 VALU ops, against 9 in integer form. This per-block
// VALU work, not the MFMA, bounds the kernel.
//
// Tiling: a workgroup of 4 R x KS waves owns a BM x 128 output tile, BM = 32 R rows (R = 1 by default; 2 and 4 are
// the taller tiles jt_gemm_bm selects), one 128-column block at BLK=128, four at BLK=32. K is walked in stages of
// 64 (BLK=32) or 128 (BLK=128) bytes per row: wave group g (4 R waves) takes stages s = g (mod KS) and stages each
// one through its own double-buffered LDS tile of BM + 128 rows (BM of A, 128 of B) with coalesced loads, issued
// two stages ahead of the MFMAs; wave w of the group computes the 32 x 32 sub-tile of rows 32 (w / 4) and columns
// 32 (w % 4) as 2 x 2 MFMA 16x16x32 tiles. The KS partial sums are added in LDS (integer addition, exact in any
// order). The summed tile is then read in a row-block layout (16 consecutive columns per lane) where the block
// quantization and the fused epilogues run:
//   MODO 0 block output | 1 raw output | 2 + residual add (soma) | 3 + ReLU^2 second output
//   4 ReLU^2 backward with H | 6 + 16-bit residual add (soma16) and its INT8 copy (para8)
// The fused epilogues compute exactly the separate ops on the quantized GEMM output (jatai_cuda.cu:195-200).
#include "jt_comum.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace gemm {
constexpr int BM = 32, BN = 128, PAD = 4;   // BM: rows of the default tile (R = 1); a tile has 32 R rows
// bytes of K per row and stage: 64 at BLK=32 (two blocks; smaller buffers, more resident waves), 128 at BLK=128
// BLK=32: 64-byte rows, unpadded, with the 8-byte chunk c of tile row r stored at chunk c ^ ((r >> 1) & 7): the
// MFMA fragment reads (16 rows x one chunk per half-wave) and the stage stores (8 rows x 8 chunks per wave) then
// touch every LDS bank once. BLK=128: 128-byte rows padded by 8 bytes.
// K-blocks held by the shift tables: all of K up to 4096 values, else chunks of 2048 values
// (ctab > 0: chunks of ctab values instead of 2048 when K is chunked anyway and ctab / blk is a multiple of 16,
// the chunked path's 16-byte exponent loads)
__host__ __device__ constexpr int bloco_tab(int nb, int blk, int ctab = 0) {
    return (nb * blk > 4096 ? (ctab > 0 && ctab < 2048 && (ctab / blk) % 16 == 0 ? ctab : 2048) : 4096) / blk;
}
// Chunk of the grouped weight-gradient launch (k_gemm_lote) past K = 4096: 1024 values, so a 32-row tile's LDS is
// 28.7 KB and five workgroups fit per CU instead of four (config 5, K = 16384: 3532 -> 3447 us; at K <= 4096 the
// single chunk of all of K measured as fast, 448 against 450 us at config 4, and is kept)
constexpr int CTAB_LOTE = 1024;
template <int BLK, int R = 1> struct Est {
    static constexpr int SK = BLK == 32 ? 64 : 128;
    static constexpr bool SWZ = BLK == 32;
    static constexpr int LD = SWZ ? SK : SK + 8;   // LDS row stride of a stage tile
    static constexpr int ROWS = 32 * R + BN;        // rows of a stage tile: 32 R of A then 128 of B
    static constexpr int STAGE = ROWS * LD;
    static constexpr int VB = SK / 8;    // bytes each of the 8 lanes of a row moves per stage
    __device__ static int pos(int r, int c) { return r * LD + 8 * (SWZ ? (c ^ ((r >> 1) & 7)) : c); }   // byte offset of chunk c
};
}

// The body of one workgroup's tile (rows row0 .., columns col0 ..), shared by k_gemm and the grouped k_gemm_lote.
// PADT: exponent rows staged with padding (below); on for the K-split and grouped kernels, where it measured faster
// (grouped launch 445 -> 435 us at config 4), off for the single-split ones, whose code it made 3-6% slower.
template <int BLK, int MODO, int KS, int R = 1, bool PADT = (KS > 1)>
__device__ __forceinline__ void gemm_corpo(const int8_t* __restrict__ A, const int8_t* __restrict__ EA, const int8_t* __restrict__ B,
                                           const int8_t* __restrict__ EB, int8_t* __restrict__ Cm, int8_t* __restrict__ CE,
                                           int* __restrict__ C32, int16_t* __restrict__ Ce, const int8_t* __restrict__ Xm,
                                           const int8_t* __restrict__ XE, int8_t* __restrict__ Om2, int8_t* __restrict__ OE2, int M, int N,
                                           int K, int kid, const int row0, const int col0, const Otim ot = Otim{}, int k_lr = 0,
                                           int ef = 0, int est = 0, int ctab = 0, int compacto = 0) {
    using gemm::BN;
    using gemm::PAD;
    using E = gemm::Est<BLK, R>;
    constexpr int SK = E::SK, LD = E::LD, STAGE = E::STAGE, VB = E::VB;
    constexpr int BM = 32 * R;                                      // tile rows
    constexpr int GT = 256 * R;                                     // threads of a K-split group (4 R waves)
    constexpr int NL = 1 + 4 / R;                                   // stage rows per thread: BM of A, then 128 of B
    constexpr int OB = BM > 64 ? BM : 64;                           // first thread of the B-row maxima (wave aligned)
    extern __shared__ __align__(16) char smem[];
    const int nb = K / BLK, ns = (K + SK - 1) / SK;
    constexpr int BPS = SK / BLK;                                   // blocks per stage
    constexpr int KST = BLK / 32;                                   // MFMA k-steps per block
    // The shift tables hold at most NBC K-blocks: all of K up to 4096 values; a longer K runs in chunks of 2048
    // values, each with its own tables (the row maxima RA, RB are over all of K). Half-size chunks keep the tables
    // of a 32-row tile at the LDS size of K = 2048, so four workgroups stay resident per CU.
    const int NBC = gemm::bloco_tab(nb, BLK, ctab);
    const int nbt = min(nb, NBC), nch = (nb + NBC - 1) / NBC;
    // LDS: RA [BM], RB [BN] int32 (live to the end); shift terms na[b][i] = ea_ib + 4 - RA_i (int32) and
    // nb[b][j] = eb_jb - RB_j (int8) of the chunk's blocks, clamped at -100 (n = na + nb <= -22 scales |p| < 2^21
    // below 1/2, i.e. to 0, as rnd(., s >= 26) does); then the stage buffers [KS][2][STAGE], which first hold the
    // chunk's raw exponent bytes and at the end the KS accumulator tiles.
    int* ra_s = reinterpret_cast<int*>(smem);
    int* rb_s = ra_s + BM;
    int* na_s = rb_s + BN;
    int8_t* nb_s = reinterpret_cast<int8_t*>(na_s + (size_t)nbt * BM);
    char* buf = reinterpret_cast<char*>(nb_s) + (((size_t)nbt * BN + 15) & ~(size_t)15);
    int8_t* st_s = reinterpret_cast<int8_t*>(buf);                 // raw exponent bytes: EA rows [BM][nbc], EB rows [BN][nbc]
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar control
    const int lr = lane & 15, lg = lane >> 4;                       // fragment row/col, k-group
    const int g = KS == 1 ? 0 : wave / (4 * R), wq = wave % (4 * R), wr = (wq >> 2) * 32, wc = (wq & 3) * 32, tg = tid & (GT - 1);
    char* meu = buf + (size_t)g * 2 * STAGE;                        // this group's two stage buffers

    // stage loads: thread tg of a group moves VB-byte vector tg % 8 of tile rows tg / 8 + BM i, i = 0 .. NL - 1
    // (rows 0 .. BM - 1 of A, then 128 of B), at lane offset (row) K + vc of its band (< 128 * 65536 = 2^23)
    const int vr = tg >> 3, vc = (tg & 7) * VB;
    int4 reg[NL], reg2[NL];                                         // two register sets: loads run two stages ahead
    // Stage loads through buffer resources of the tile's A rows and B rows (bounds: the tile's own bytes, so no
    // access leaves them): the stage offset is the scalar operand, the lane offsets stay fixed, and a stage takes no
    // vector address arithmetic. The last stage may extend past K (nb not a multiple of the blocks per stage): its
    // vectors past K re-read the row's last vector instead (those bytes land in blocks >= nb, never computed).
    const auto rsA = __builtin_amdgcn_make_buffer_rsrc((void*)(A + (size_t)row0 * K), (short)0, BM * K, 0x00020000);
    const auto rsB = __builtin_amdgcn_make_buffer_rsrc((void*)(B + (size_t)col0 * K), (short)0, BN * K, 0x00020000);
    int voff[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) voff[i] = (i == 0 ? vr : BM * (i - 1) + vr) * K + vc;
    auto carrega = [&](int4& r, int i, int vo, int so) {
        if constexpr (VB == 16) {
            const v4i t = __builtin_amdgcn_raw_buffer_load_b128(i == 0 ? rsA : rsB, vo, so, 0);
            r = make_int4(t[0], t[1], t[2], t[3]);
        } else {
            typedef int v2i __attribute__((ext_vector_type(2)));
            const v2i t = __builtin_amdgcn_raw_buffer_load_b64(i == 0 ? rsA : rsB, vo, so, 0);
            r = make_int4(t[0], t[1], 0, 0);
        }
    };
    auto busca = [&](int st, int4 (&r)[NL]) {
        const int o = __builtin_amdgcn_readfirstlane(st * SK);
        if (o + SK <= K) {
#pragma unroll
            for (int i = 0; i < NL; i++) carrega(r[i], i, voff[i], o);
        } else {
            const int d = min(o + vc, K - VB) - vc;
#pragma unroll
            for (int i = 0; i < NL; i++) carrega(r[i], i, voff[i] + d, 0);
        }
    };
    auto guarda = [&](int par, const int4 (&r)[NL]) {
        char* d = meu + par * STAGE;
#pragma unroll
        for (int i = 0; i < NL; i++) {
            if constexpr (VB == 16) {
                int2* q = reinterpret_cast<int2*>(d + (vr + BM * i) * LD + vc);
                q[0] = make_int2(r[i].x, r[i].y);
                q[1] = make_int2(r[i].z, r[i].w);
            } else {
                *reinterpret_cast<int2*>(d + E::pos(vr + BM * i, vc >> 3)) = make_int2(r[i].x, r[i].y);
            }
        }
    };
    // output-stage coordinates: row orow, columns oc .. oc + EV - 1. The block-output epilogues (modes 0, 2, 3, 4,
    // 6) run on every thread, EV = 16 / KS values each (all K-split groups share the partial sums and the
    // quantization); the raw-output and optimizer epilogues (modes 1, 5) on the first group, 16 values each.
    constexpr int EV = (MODO == 1 || MODO == 5) ? 16 : 16 / KS, LPR_ = 128 / EV;
    const int orow = (tid / LPR_) & (BM - 1), oc = (tid % LPR_) * EV;
    const bool saida = EV < 16 || tid < GT;
    // Several chunks: RA and RB first, by one pass over the exponent rows in global memory (rows of nb bytes, nb a
    // multiple of 16 there: 16-byte loads). One chunk: from the staged exponents, below.
    if (nch > 1) {
        const int8_t* er = tid < BM ? EA + (size_t)(row0 + tid) * nb
                                    : (tid >= OB && tid < OB + BN) ? EB + (size_t)(col0 + tid - OB) * nb : nullptr;
        if (er) {
            int m = -128;
            for (int v = 0; v < nb / 16; v++) {
                const int4 t = reinterpret_cast<const int4*>(er)[v];
                m = max(m, max(max(max_i8x4(t.x), max_i8x4(t.y)), max(max_i8x4(t.z), max_i8x4(t.w))));
            }
            if (tid < BM) ra_s[tid] = m;
            else rb_s[tid - OB] = m;
        }
    }
    // shift tables of K-blocks b0 .. b0 + nbc - 1 from the staged exponent bytes (rows of nbc bytes); then the
    // stage buffers are free again
    // A thread's row r = tid % 32 and column c = tid % 128 are the same in every iteration, so their maxima are read
    // once; the exponent bytes of U iterations are read before any table entry is written (the writes could alias
    // the reads for the compiler, which would otherwise wait on every read).
    // The staged rows are sst bytes apart: with PADT, nbc + 4 when nbc is a multiple of 16, an odd number of 4-byte words, so
    // the byte reads below (consecutive threads, consecutive rows) fall in different LDS banks; rows nbc bytes
    // apart (a multiple of 64 at K >= 2048) put a wave's reads in two banks.
    auto desloca_tab = [&](int nbc, int sst) {
        const int r = tid & (BM - 1), c = tid & (BN - 1);
        const int ra4 = 4 - ra_s[r], rbn = -rb_s[c];
        const int8_t* ea = st_s + r * sst;
        const int8_t* eb = st_s + (BM + c) * sst;
        constexpr int U = 4, SA = GT * KS / BM, SB = GT * KS / BN;   // SA = 8 KS, SB = 2 R KS
        for (int b0 = tid / BM; b0 < nbc; b0 += U * SA) {           // entries b * BM + r
            int e[U];
#pragma unroll
            for (int u = 0; u < U; u++) e[u] = b0 + u * SA < nbc ? (int)ea[b0 + u * SA] : 0;
#pragma unroll
            for (int u = 0; u < U; u++)
                if (b0 + u * SA < nbc) na_s[(b0 + u * SA) * BM + r] = max(e[u] + ra4, -100);
        }
        for (int b0 = tid >> 7; b0 < nbc; b0 += 2 * U * SB) {       // entries b * BN + c
            int e[2 * U];
#pragma unroll
            for (int u = 0; u < 2 * U; u++) e[u] = b0 + u * SB < nbc ? (int)eb[b0 + u * SB] : 0;
#pragma unroll
            for (int u = 0; u < 2 * U; u++)
                if (b0 + u * SB < nbc) nb_s[(b0 + u * SB) * BN + c] = (int8_t)max(e[u] + rbn, -100);
        }
        __syncthreads();
    };
    // one chunk (K <= 4096): the tile's BM rows of A and 128 rows of B are two contiguous spans (BM nb and 128 nb
    // bytes, multiples of 16): 16-byte loads in rounds of 4, all issued before the stores; indices past the span
    // re-read its last vector and store it to a junk slot after the span, so neither side branches. RA and RB
    // come from the staged bytes.
    auto tabelas_unica = [&]() {
        const int nva = BM * nb / 16, nvt = (BM + BN) * nb / 16;
        const int4* ga = reinterpret_cast<const int4*>(EA + (size_t)row0 * nb);
        const int4* gb = reinterpret_cast<const int4*>(EB + (size_t)col0 * nb);
        // rows of whole vectors, 32 bytes or more (the ones that fall in 4 or fewer banks): staged sst1 bytes apart;
        // at 16 bytes (8 banks) the padding's split stores cost more than the conflicts (K = 512: 2-5% slower)
        const bool pad = PADT && nb % 16 == 0 && nb >= 32;
        const int q = pad ? nb / 16 : 1, sst1 = pad ? nb + 4 : nb;
        for (int v0 = tid; v0 < nvt; v0 += 4 * GT * KS) {
            int4 t[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int v = min(v0 + k * GT * KS, nvt - 1);
                t[k] = v < nva ? ga[v] : gb[v - nva];
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int v = min(v0 + k * GT * KS, nvt);
                if (pad) {                                            // v = nvt: the junk row BM + BN
                    const int r = v / q;
                    int* d = reinterpret_cast<int*>(st_s + (size_t)r * sst1 + 16 * (v - r * q));
                    d[0] = t[k].x; d[1] = t[k].y; d[2] = t[k].z; d[3] = t[k].w;
                } else {
                    *reinterpret_cast<int4*>(st_s + (size_t)v * 16) = t[k];
                }
            }
        }
        __syncthreads();
        // RA, RB: 4 exponent bytes per LDS read from padded rows, 16 from unpadded rows of whole vectors, else 1
        const int8_t* er = tid < BM ? st_s + tid * sst1 : (tid >= OB && tid < OB + BN) ? st_s + (BM + tid - OB) * sst1 : nullptr;
        if (er) {
            int m = -128;
            if (pad) {
                for (int b = 0; b < nb; b += 4) m = max(m, max_i8x4(*reinterpret_cast<const int*>(er + b)));
            } else if (nb % 16 == 0) {
                for (int b = 0; b < nb; b += 16) {
                    const int4 t = *reinterpret_cast<const int4*>(er + b);
                    m = max(m, max(max(max_i8x4(t.x), max_i8x4(t.y)), max(max_i8x4(t.z), max_i8x4(t.w))));
                }
            } else {
                for (int b = 0; b < nb; b++) m = max(m, (int)er[b]);
            }
            if (tid < BM) ra_s[tid] = m;
            else rb_s[tid - OB] = m;
        }
        __syncthreads();
        desloca_tab(nb, sst1);
    };
    // one chunk whose exponent rows are whole 16-byte vectors, at most 8 per row (K <= 4096): no staging. A row is
    // taken by LR = 1, 2, 4 or 8 consecutive lanes (the power of two at or above its nb / 16 vectors), each loading
    // one vector into registers; the row maximum is a reduction over those lanes, and each lane writes its 16 table
    // entries (and the maximum) straight into LDS. All loads are issued before the first reduction. One barrier
    // (the caller's, after the first stage's store) publishes the tables instead of three.
    auto tabelas_diretas = [&]() {
        const int q = nb / 16, LR = q <= 1 ? 1 : q <= 2 ? 2 : q <= 4 ? 4 : 8;
        const int itens = (BM + BN) * LR, NT = GT * KS;
        constexpr int KMAX = ((32 * R + 128) * 8 + 256 * R * KS - 1) / (256 * R * KS);   // rounds for LR = 8: 5 at most
        int4 t[KMAX];
#pragma unroll
        for (int k = 0; k < KMAX; k++) {
            const int it = tid + k * NT, row = it / LR, j = it % LR;
            t[k] = make_int4(0x80808080, 0x80808080, 0x80808080, 0x80808080);   // -128: neutral for the maximum
            if (it < itens && j < q)
                t[k] = *reinterpret_cast<const int4*>((row < BM ? EA + (size_t)(row0 + row) * nb : EB + (size_t)(col0 + row - BM) * nb) + 16 * j);
        }
#pragma unroll
        for (int k = 0; k < KMAX; k++) {
            if (k * NT >= itens) break;                              // uniform
            const int it = tid + k * NT, row = it / LR, j = it % LR;
            int m = max(max(max_i8x4(t[k].x), max_i8x4(t[k].y)), max(max_i8x4(t[k].z), max_i8x4(t[k].w)));
            m = LR == 1 ? m : LR == 2 ? g_max<2>(m) : LR == 4 ? g_max<4>(m) : g_max<8>(m);
            if (it >= itens || j >= q) continue;
            const int w4[4] = {t[k].x, t[k].y, t[k].z, t[k].w};
            if (row < BM) {
                if (j == 0) ra_s[row] = m;
                const int ra4 = 4 - m;
#pragma unroll
                for (int u = 0; u < 16; u++) na_s[(16 * j + u) * BM + row] = max((int)(int8_t)(w4[u >> 2] >> (8 * (u & 3))) + ra4, -100);
            } else {
                const int c = row - BM;
                if (j == 0) rb_s[c] = m;
#pragma unroll
                for (int u = 0; u < 16; u++) nb_s[(16 * j + u) * BN + c] = (int8_t)max((int)(int8_t)(w4[u >> 2] >> (8 * (u & 3))) - m, -100);
            }
        }
    };
    // several chunks: 160 row segments of nbc bytes (a multiple of 16) at column b0 of rows of nb bytes, one
    // 16-byte vector at a time (this runs between chunks, with the accumulators live)
    auto tabelas_parte = [&](int b0, int nbc) {
        const int vpr = nbc / 16, sst = PADT ? nbc + 4 : nbc;
        for (int v = tid; v < (BM + BN) * vpr; v += GT * KS) {
            const int r = v / vpr, k = v - r * vpr;
            const int8_t* e = r < BM ? EA + (size_t)(row0 + r) * nb : EB + (size_t)(col0 + r - BM) * nb;
            const int4 t = *reinterpret_cast<const int4*>(e + b0 + 16 * k);
            if constexpr (PADT) {
                int* d = reinterpret_cast<int*>(st_s + (size_t)r * sst + 16 * k);
                d[0] = t.x; d[1] = t.y; d[2] = t.z; d[3] = t.w;
            } else {
                *reinterpret_cast<int4*>(st_s + (size_t)r * sst + 16 * k) = t;
            }
        }
        __syncthreads();
        desloca_tab(nbc, sst);
    };
    int b0 = 0;                                                     // first K-block of the current chunk
    // chunk 0, before the accumulators are live: its first two stages in flight during the exponent staging
    if (g < min(ns, NBC / BPS)) busca(g, reg);
    if (g + KS < min(ns, NBC / BPS)) busca(g + KS, reg2);
    if (nch == 1 && nb % 16 == 0 && nb <= 128) tabelas_diretas();
    else if (nch == 1) tabelas_unica();
    else tabelas_parte(0, NBC);
    if (g < min(ns, NBC / BPS)) guarda(0, reg);
    __syncthreads();

    int acc[2][2][4] = {};
    int fora = 0;                                                   // bit 8 ti + 4 tj + i: acc[ti][tj][i] out of range
    // stage k of this group in a chunk (k = 0, 1, ...) is stage gs + k KS, held in buffer k % 2. In iteration k the loads of
    // stage k + 2 are issued, stage k is computed, and stage k + 1 (loaded during iteration k - 1) is stored -- into
    // the buffer of stage k - 1, which every wave finished reading before the barrier that ended iteration k - 1.
    // Each block's MFMAs are followed by its rounding: the MFMA latency runs under the other resident waves' VALU
    // work, and only one block's products are live (the fp64 rounding's temporaries need the registers).
    auto produtos = [&](const char* tile, int bl, v4i (&p)[2][2]) {
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
            for (int tj = 0; tj < 2; tj++) p[ti][tj] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < KST; k++) {
            const int ch = (bl * KST + k) * 4 + lg;                   // 8-byte chunk of K within the stage
            long fa[2], fb[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                fa[t] = *reinterpret_cast<const long*>(tile + E::pos(wr + 16 * t + lr, ch));
                fb[t] = *reinterpret_cast<const long*>(tile + E::pos(BM + wc + 16 * t + lr, ch));
            }
#pragma unroll
            for (int ti = 0; ti < 2; ti++)
#pragma unroll
                for (int tj = 0; tj < 2; tj++) p[ti][tj] = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa[ti], fb[tj], p[ti][tj], 0, 0, 0);
        }
    };
    // rnd(p << 4, sa + sb) from the row term n = 4 - sa and the column scale c = 2^-sb (see the head of this file)
    auto rnd_fma = [](int p, int n, double c) { return __double2loint(__builtin_fma(ldexp((double)p, n), c, 0x1.8p52)); };
    auto escala = [](int nbv) { return __hiloint2double((1023 + nbv) << 20, 0); };
    auto arredonda = [&](int b, const v4i (&p)[2][2]) {
        const int bt = b - b0;                                      // block index in the chunk's tables
        const v4i na0 = *reinterpret_cast<const v4i*>(na_s + bt * BM + wr + 4 * lg);
        const v4i na1 = *reinterpret_cast<const v4i*>(na_s + bt * BM + wr + 16 + 4 * lg);
        const double cb0 = escala(nb_s[bt * BN + wc + lr]), cb1 = escala(nb_s[bt * BN + wc + 16 + lr]);
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
            for (int tj = 0; tj < 2; tj++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[ti][tj][i] += rnd_fma(p[ti][tj][i], ti ? na1[i] : na0[i], tj ? cb1 : cb0);
    };
    auto calcula = [&](const char* tile, int st) {
#pragma unroll
        for (int bl = 0; bl < BPS; bl++) {
            if (st * BPS + bl >= nb) break;
            v4i p[2][2];
            produtos(tile, bl, p);
            arredonda(st * BPS + bl, p);
        }
    };
    for (int c = 0; c < nch; c++) {
        b0 = c * NBC;
        const int nbc = min(NBC, nb - b0);
        const int s0 = b0 / BPS, s1 = min(ns, (b0 + nbc + BPS - 1) / BPS);   // the chunk's stages
        const int gs = s0 + g;                                      // this group's first stage
        if (c > 0) {                                                // chunk 0 was staged above
            if (gs < s1) busca(gs, reg);
            if (gs + KS < s1) busca(gs + KS, reg2);
            tabelas_parte(b0, nbc);
            if (gs < s1) guarda(0, reg);
            __syncthreads();
        }
        const int nk = gs < s1 ? (s1 - gs + KS - 1) / KS : 0;       // stages of this group in the chunk
        for (int k = 0; k < nk; k += 2) {
            // even k: new loads into reg (its stage is stored), the pending stage k + 1 sits in reg2
            if (k + 2 < nk) busca(gs + (k + 2) * KS, reg);
            calcula(meu, gs + k * KS);
            if (k + 1 < nk) guarda(1, reg2);
            __syncthreads();
            if (k + 1 >= nk) break;
            // odd k + 1: the stage k + 2 loads sit in reg; new loads into reg2
            if (k + 3 < nk) busca(gs + (k + 3) * KS, reg2);
            calcula(meu + STAGE, gs + (k + 1) * KS);
            if (k + 2 < nk) guarda(0, reg);
            __syncthreads();
        }
        // groups with fewer stages still take part in every barrier of the loop above
        for (int k = nk; k < (s1 - s0 + KS - 1) / KS; k++) __syncthreads();
        // Past 4096 values of K the int32 accumulator has no a-priori bound: 4096 values of K add less than 2^30
        // (4096 / BLK blocks of |rnd(p << 4, s)| < 2^23 BLK / 32), so a partial sum kept below 2^30 / KS at every
        // multiple of 4096 values (every second chunk) and at the end can neither wrap in between nor in the sum of
        // the KS partials; one that is not is reported.
        // (the violations are collected as bits and reported after the loop: a call here, with the accumulators
        // and both stage register sets live, would make the compiler keep registers in scratch)
        if (nch > 1 && ((b0 + nbc) * BLK % 4096 == 0 || c == nch - 1)) {
            constexpr int T = LIM / KS;
#pragma unroll
            for (int ti = 0; ti < 2; ti++)
#pragma unroll
                for (int tj = 0; tj < 2; tj++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        fora |= (int)(acc[ti][tj][i] >= T || acc[ti][tj][i] <= -T) << (8 * ti + 4 * tj + i);
        }
    }

    // ---- output stage: KS partial tiles to LDS, summed while read back in the row-block layout. The X operand
    // of modes 2 and 4 is read here, not before the K loop, so its 16 registers do not cost a resident wave.
    const size_t o = (size_t)(row0 + orow) * N + col0 + oc;
    const size_t oe = (size_t)(row0 + orow) * (N / BLK) + (col0 + oc) / BLK;
    int xin[EV], exin = 0;
    if constexpr (MODO == 2 || MODO == 4) {
        if (saida) { le_i8(Xm + o, xin); exin = XE[oe]; }
    }
    if constexpr (MODO == 6) {                                     // the R16 residual (int16 mantissas)
        if (saida) { le_i16(reinterpret_cast<const int16_t*>(Xm) + o, xin); exin = XE[oe]; }
    }
    int base[EV];
    if (saida) {
        const int ra = ra_s[orow];
#pragma unroll
        for (int j = 0; j < EV; j++) base[j] = ra + rb_s[oc + j] - 4;
    }
    int* acc_s = reinterpret_cast<int*>(buf);                      // [KS][BM][BN + PAD]
    constexpr int TILE = BM * (BN + PAD);
#pragma unroll
    for (int ti = 0; ti < 2; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc_s[g * TILE + (wr + 16 * ti + 4 * lg + i) * (BN + PAD) + wc + 16 * tj + lr] = acc[ti][tj][i];
    if (fora) {                                                     // K > 4096 only: an accumulator out of range
        const int e = __builtin_ctz(fora), ti = e >> 3, tj = (e >> 2) & 1, i = e & 3;
        reporta(E_ACUM, kid, (long long)(row0 + wr + 16 * ti + 4 * lg + i) * N + col0 + wc + 16 * tj + lr,
                acc_s[g * TILE + (wr + 16 * ti + 4 * lg + i) * (BN + PAD) + wc + 16 * tj + lr], -3);
    }
    OtimEnt<16> otx;                                               // mode 5: the optimizer's inputs, in flight during the LDS round trip
    if constexpr (MODO == 5) {
        if (tid < GT) otx = otim_le<16>(ot, (long long)o, (long long)(o / BLK), ef);
    }
    __syncthreads();
    if constexpr (MODO == 1) {
        // raw output in 16-byte pieces: thread t writes columns 4 (t % 32) .. + 3 of rows t / 32 + 8 R k, k = 0 .. 3
        // (a wave: two rows of 512 contiguous bytes of C32 and 256 of Ce)
        // compacto: the exponent of (i, j) is RA_i + RB_j - 4 (RA, RB maxima of int8 exponents, so never below the
        // -30000 clamp), stored as the vectors Ce[i] = RA_i (i < M) and Ce[M + j] = RB_j - 4, written by the tiles of
        // the first column and of the first row: 2 (M + N) bytes instead of 2 M N
        typedef short s4_t __attribute__((ext_vector_type(4)));
        if (tid < GT) {
            const int c = (tid & 31) * 4;
            int rbc[4];
#pragma unroll
            for (int x = 0; x < 4; x++) rbc[x] = rb_s[c + x] - 4;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int r = (tid >> 5) + 8 * R * k;
                v4i t = *reinterpret_cast<const v4i*>(acc_s + r * (BN + PAD) + c);
#pragma unroll
                for (int q = 1; q < KS; q++) t += *reinterpret_cast<const v4i*>(acc_s + q * TILE + r * (BN + PAD) + c);
                const size_t oo = (size_t)(row0 + r) * N + col0 + c;
                *reinterpret_cast<v4i*>(C32 + oo) = t;
                if (compacto) continue;
                const int ra = ra_s[r];
                *reinterpret_cast<s4_t*>(Ce + oo) = s4_t{(short)max(-30000, ra + rbc[0]), (short)max(-30000, ra + rbc[1]),
                                                         (short)max(-30000, ra + rbc[2]), (short)max(-30000, ra + rbc[3])};
            }
            if (compacto) {
                if (col0 == 0 && tid < BM) Ce[row0 + tid] = (short)ra_s[tid];
                if (row0 == 0 && tid < BN) Ce[M + col0 + tid] = (short)(rb_s[tid] - 4);
            }
        }
        return;
    } else {
        if (!saida) return;
        int v[EV];
#pragma unroll
        for (int j = 0; j < EV; j += 4) {
            v4i t = *reinterpret_cast<const v4i*>(acc_s + orow * (BN + PAD) + oc + j);
#pragma unroll
            for (int q = 1; q < KS; q++) t += *reinterpret_cast<const v4i*>(acc_s + q * TILE + orow * (BN + PAD) + oc + j);
            v[j] = t[0]; v[j + 1] = t[1]; v[j + 2] = t[2]; v[j + 3] = t[3];
        }
        constexpr int LPB = BLK / EV;
        const bool lider = (tid & (LPB - 1)) == 0;
        // KS = 1, BLK = 32 (every thread here, EV = 16, so the barriers are uniform): the block-format output q (its
        // block's exponent Eq) also written transposed, Yt [N, M] blocked along M. The tile's BM rows are R blocks of
        // each of its 128 columns: the same requantization as k_transpoe (quant(m^T, expand(E)^T), ops.py:121-123),
        // from the quantized tile staged in LDS.
        // LDS layout: mantissa rows of BN bytes whose 16-byte chunk j sits at chunk j ^ ((row / 16) % 8), and exponent
        // rows 5 bytes apart: the column reads below (8 threads of a column each take rows 16 pt .. 16 pt + 15, pt =
        // 0 .. 7) then fall in 8 distinct chunks and banks instead of one bank 8 times over.
        auto escreve_t = [&](const int8_t (&q)[EV], int Eq, int8_t* __restrict__ Yt, int8_t* __restrict__ YEt) {
            if constexpr (KS == 1 && BLK == 32) {
                constexpr int ES = 5;
                int8_t* qs = reinterpret_cast<int8_t*>(buf);           // [BM][BN] mantissas, chunk-swizzled
                int8_t* es = qs + BM * BN;                              // [BM][ES] exponents
                __syncthreads();                                        // acc_s fully read before the reuse
                grava_i8(qs + orow * BN + 16 * ((oc >> 4) ^ ((orow >> 4) & 7)), q);
                if (lider) es[orow * ES + oc / 32] = (int8_t)Eq;
                __syncthreads();
                // column c, rows 16 pt .. 16 pt + 15 (2 R threads per column; lanes 2j, 2j + 1 hold one block)
                const int c = tid / (2 * R), pt = tid % (2 * R);
                const int8_t* qc = qs + 16 * ((c >> 4) ^ (pt & 7)) + (c & 15);
                int tv[16], te[16];
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    const int r = 16 * pt + k;
                    tv[k] = qc[r * BN];
                    te[k] = es[r * ES + (c >> 5)];
                }
                int8_t t8[16];
                const long long ot = (long long)(col0 + c) * M + row0 + 16 * pt;
                const int Et = quant8_d<16, 2>(tv, te, t8, kid, ot);   // int8 exponents
                grava_i8(Yt + ot, t8);
                if ((pt & 1) == 0) YEt[(size_t)(col0 + c) * (M / 32) + row0 / 32 + (pt >> 1)] = (int8_t)Et;
            }
        };
        if constexpr (MODO == 5) {                                 // weight gradient straight into momento + peso
            int eg[16];
#pragma unroll
            for (int j = 0; j < 16; j++) eg[j] = max(-30000, base[j]);   // the raw output's int16 exponent
            int qw[16], Ew;
            otim_valores<16, LPB>(v, eg, otx, ot, (long long)o, (long long)(o / BLK), lider, k_lr, ef, kid, qw, Ew);
            return;
        }
        int8_t m[EV];
        const int E = quant8_d<EV, LPB>(v, base, m, kid, o);        // |base| <= 260
        if constexpr (MODO == 0 || MODO == 3) {
            grava_i8(Cm + o, m);
            if (lider) CE[oe] = (int8_t)E;
        }
        if constexpr (MODO == 3) {                                 // a = relu2(h): max(m, 0)^2, exponent 2E
            int a[EV];
#pragma unroll
            for (int j = 0; j < EV; j++) { const int h = max((int)m[j], 0); a[j] = h * h; }
            int8_t q[EV];
            const int Ea = quant8_comum<EV, LPB>(a, 2 * E, q);
            if (Ea > 126 && lider) reporta(E_EXP, kid, (long long)o, Ea, -7);
            grava_i8(Om2 + o, q);
            if (lider) OE2[oe] = (int8_t)Ea;
            if (C32 != nullptr) escreve_t(q, Ea, reinterpret_cast<int8_t*>(C32), reinterpret_cast<int8_t*>(Ce));   // T(a)
        }
        if constexpr (MODO == 6) {
            // z16 = soma16(X16, C) (jatai_cuda.cu:514-531: ec = max(xE + 15, E + 7) - 28, zero blocks add 0, a
            // 15-bit block quantization) into Cm (int16 mantissas) and CE, then y8 = para8(z16) (jatai_cuda.cu:
            // 501-513) into Om2, OE2: what jt_soma16 and jt_para8 compute from the stored tensors. The exponents
            // are taken as stored (int8), so even an out-of-range one gives the separate launches' bits.
            const int ey = (int)(int8_t)E, ec = max(exin + 15, ey + 7) - 28;
            const Desl dx(ec - exin), dm(ec - ey);                 // left shifts keep |values| below 2^28
            const int mx = exin == E_ZERO ? 0 : -1, mm = ey == E_ZERO ? 0 : -1;
            int s[EV], q[EV];
#pragma unroll
            for (int j = 0; j < EV; j++) s[j] = (dx(xin[j]) & mx) + (dm((int)m[j]) & mm);
            const int Ez = quant_u<EV, LPB, true, 15, 32767>(s, ec, q, kid + 1, (long long)o);   // soma16's launch id
            int16_t z[EV];
#pragma unroll
            for (int j = 0; j < EV; j++) z[j] = (int16_t)q[j];
            grava_i16(reinterpret_cast<int16_t*>(Cm) + o, z);
            if (lider) CE[oe] = (int8_t)Ez;
            int8_t y[EV];
            const int Ey = quant8_u8<EV, LPB>(q, (int)(int8_t)Ez, y, kid + 2, (long long)o);     // para8's launch id
            grava_i8(Om2 + o, y);
            if (lider) OE2[oe] = (int8_t)Ey;
        }
        if constexpr (MODO == 2) {                                 // z = soma(X, C): ec = max(xE, E) - 21
            int s[EV];
            const int ec = max(exin, E) - 21;
            const Desl dx(ec - exin), dm(ec - E);                  // exact left shifts or roundings, |s| <= 2^28
#pragma unroll
            for (int j = 0; j < EV; j++) s[j] = dx(xin[j]) + dm((int)m[j]);
            int8_t q[EV];
            int Ez;
            if (est) {                                             // stochastic rounding (jt_res_estocastico)
                // seeds as the reference's epilogue lays out a 128-column tile: the value at tile column c has seed
                // 8 (flat index of column c & 60 of its row) + (c & 3) + 4 (c >= 64), in 32-bit arithmetic
                uint32_t h[EV];
#pragma unroll
                for (int j = 0; j < EV; j++) {
                    const int c = oc + j;
                    h[j] = (uint32_t)((size_t)(row0 + orow) * N + col0 + (c & 60)) * 8u + (uint32_t)((c & 3) + 4 * ((c >> 6) & 1));
                }
                Ez = quant8_est<EV, LPB>(s, ec, q, h);
            } else {
                Ez = quant8_comum<EV, LPB>(s, ec, q);
            }
            if (Ez > 126 && lider) reporta(E_EXP, kid, (long long)o, Ez, -6);
            grava_i8(Cm + o, q);
            if (lider) CE[oe] = (int8_t)Ez;
        }
        if constexpr (MODO == 4) {                                 // gh = C * 2 max(H, 0), exponent E + eh
            int s[EV];
#pragma unroll
            for (int j = 0; j < EV; j++) s[j] = (int)m[j] * max(xin[j], 0) * 2;
            int8_t q[EV];
            const int Eg = quant8_comum<EV, LPB>(s, E + exin, q);
            if (Eg > 126 && lider) reporta(E_EXP, kid, (long long)o, Eg, -8);
            grava_i8(Cm + o, q);
            if (lider) CE[oe] = (int8_t)Eg;
            if (Om2 != nullptr) escreve_t(q, Eg, Om2, OE2);            // T(gh)
        }
    }
}

// jt_res_estocastico's switch, as in the reference a device global (jatai_cuda.cu:146) read when a mode-2 kernel
// runs, so a captured graph follows the value set before each replay.
__device__ int g_res_est = 0;

// Tile of workgroup id in a grid of n workgroups. The dispatcher deals workgroups to the 8 XCDs in turn (id mod 8),
// each XCD with its own L2. A grid of at most 1024 workgroups is resident at once; there XCD x takes the x-th
// eighth of the tiles in row-major order, so the column tiles of a row band (which read the same A rows) share one
// L2 instead of four (at config 4: ReLU^2 GEMM 19.8 -> 18.8 us, residual-add GEMM 16.8 -> 16.4). Larger grids
// keep the plain order, which measured as fast or faster there. A bijection whenever n is a multiple of 8.
__device__ __forceinline__ int tile_xcd(int id, int n) {
    if (n > 1024 || (n & 7)) return id;
    return (id & 7) * (n >> 3) + (id >> 3);
}

template <int BLK, int MODO, int KS, int R = 1>
__global__ void __launch_bounds__(256 * R * KS) __attribute__((amdgpu_waves_per_eu(4))) k_gemm(const int8_t* __restrict__ A, const int8_t* __restrict__ EA, const int8_t* __restrict__ B,
                                                   const int8_t* __restrict__ EB, int8_t* __restrict__ Cm, int8_t* __restrict__ CE,
                                                   int* __restrict__ C32, int16_t* __restrict__ Ce, const int8_t* __restrict__ Xm,
                                                   const int8_t* __restrict__ XE, int8_t* __restrict__ Om2, int8_t* __restrict__ OE2, int M,
                                                   int N, int K, int kid) {
    const int nx = gridDim.x, t = tile_xcd(blockIdx.y * nx + blockIdx.x, nx * gridDim.y);
    gemm_corpo<BLK, MODO, KS, R>(A, EA, B, EB, Cm, CE, C32, Ce, Xm, XE, Om2, OE2, M, N, K, kid, (t / nx) * 32 * R, (t % nx) * gemm::BN,
                              Otim{}, 0, 0, MODO == 2 ? g_res_est : 0);
}

// Many raw-output GEMMs with one K in one launch (the weight gradients of a step: K = tokens). The list travels
// by value in the kernel arguments; GEMM i owns the workgroups [ini_i, ini_{i+1}) of a 1-D grid, row-major over
// its (M / 32 R) x (N / 128) tiles. Same tiles, same arithmetic as k_gemm<BLK, 1, KS, R>.
constexpr int LOTE_G = 64;                  // 3856 bytes of kernel arguments: every weight gradient of a step in one launch
static_assert(sizeof(int8_t*) * 6 * LOTE_G + sizeof(int) * (3 * LOTE_G + 4) <= 4096, "kernel argument limit");
struct LoteG {
    const int8_t* A[LOTE_G];
    const int8_t* EA[LOTE_G];
    const int8_t* B[LOTE_G];
    const int8_t* EB[LOTE_G];
    int* C32[LOTE_G];
    int16_t* Ce[LOTE_G];
    int M[LOTE_G], N[LOTE_G], ini[LOTE_G + 1];
    int n, K;
    int compacto;                           // exponents as row and column vectors (the mode-1 epilogue of gemm_corpo)
};

template <int BLK, int KS, int R = 1>
__global__ void __launch_bounds__(256 * R * KS) __attribute__((amdgpu_waves_per_eu(4))) k_gemm_lote(const LoteG L, int kid) {
    const int t = blockIdx.x;
    int i = 0;                                                      // uniform: kernel arguments, scalar loads
    for (int s = 32; s; s >>= 1)
        if (i + s < L.n && L.ini[i + s] <= t) i += s;
    const int local = t - L.ini[i], ntx = L.N[i] / gemm::BN;
    gemm_corpo<BLK, 1, KS, R, true>(L.A[i], L.EA[i], L.B[i], L.EB[i], nullptr, nullptr, L.C32[i], L.Ce[i], nullptr, nullptr, nullptr, nullptr,
                                    L.M[i], L.N[i], L.K, kid + i, (local / ntx) * 32 * R, (local % ntx) * gemm::BN, Otim{}, 0, 0, 0,
                                    gemm::CTAB_LOTE, L.compacto);
}

// The weight gradients of a step with the optimizer in the epilogue (mode 5): GEMM i's tile goes through
// momento + peso of tensor i (ops.py:273-290) instead of to memory -- the raw gradient is never stored.
constexpr int LOTE_GO = 32;
struct LoteGO {
    const int8_t* A[LOTE_GO];
    const int8_t* EA[LOTE_GO];
    const int8_t* B[LOTE_GO];
    const int8_t* EB[LOTE_GO];
    Otim ot[LOTE_GO];
    int M[LOTE_GO], N[LOTE_GO], ini[LOTE_GO + 1];
    int n, K;
};

template <int BLK, int KS, int R = 1>
__global__ void __launch_bounds__(256 * R * KS) __attribute__((amdgpu_waves_per_eu(4))) k_gemm_otim_lote(const LoteGO L, int k_lr, int ef, int kid) {
    const int t = blockIdx.x;
    int i = 0;
    for (int s = 16; s; s >>= 1)
        if (i + s < L.n && L.ini[i + s] <= t) i += s;
    const int local = t - L.ini[i], ntx = L.N[i] / gemm::BN;
    gemm_corpo<BLK, 5, KS, R>(L.A[i], L.EA[i], L.B[i], L.EB[i], nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, L.M[i],
                              L.N[i], L.K, kid + i, (local / ntx) * 32 * R, (local % ntx) * gemm::BN, L.ot[i], k_lr, ef);
}

// dynamic LDS bytes for nb K-blocks, KS K-splits and tiles of 32 R rows
static inline size_t gemm_lds(int nb, int ks, int blk, int R = 1, int ctab = 0) {
    using gemm::BN;
    using gemm::PAD;
    const int bm = 32 * R;
    nb = std::min(nb, gemm::bloco_tab(nb, blk, ctab));              // the shift tables hold one chunk of K
    const size_t fixo = (size_t)(bm + BN) * 4 + (size_t)nb * bm * 4 + (((size_t)nb * BN + 15) & ~(size_t)15);
    const size_t stage = (size_t)(32 * R + BN) * (blk == 32 ? gemm::Est<32>::LD : gemm::Est<128>::LD);
    size_t area = (size_t)ks * 2 * stage;
    const size_t exp_bruto = (size_t)(nb + 4) * (bm + BN + 1) + 16;   // staged rows nb + 4 bytes apart, and a junk row
    const size_t acc = (size_t)ks * bm * (BN + PAD) * 4;
    if (exp_bruto > area) area = exp_bruto;
    if (acc > area) area = acc;
    return fixo + area;
}
