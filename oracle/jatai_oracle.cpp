// CPU oracle of the Jatai integer training hot path -- TEST INFRASTRUCTURE ONLY.
//
// A scalar int64 restatement of the reference's executable specification `OpsRef` (jatai_cuda/ops.py:34-290),
// with the block size `blk` as a parameter (the reference fixes BLK = 128, ops.py:17), plus the three 16-bit
// residual ops that have no spec and are restated from their kernel text (jatai_cuda/jatai_cuda.cu:446-531).
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
// checker or the timed CPU baseline; the product path (jatai_amd/) never calls it.
//
// Pinning (each function's checks live in tests/test_oracle.py):
//   bitlen, rnd, exp_int, isqrt ........ reference golden vectors (primitives.json) + closed forms
//   gemm (blk 32 / 128), quant, soma, relu2, relu2_back, transpoe, embed, um_quente, rms, rms_back,
//   atencao / atencao_back (hd = 4), softmax_ce, momento, peso ...... reference golden vectors
//                                        (ops_blk128.json, ops_blk32.json, config1.json, trace_r.json)
//   atencao / atencao_back at hd > 4 (declared extension) ...... reduction to the golden-pinned hd = 4 code with
//                                        the data in dims 0-3, 32-35 or 60-63 (the head's second block, its first
//                                        all-zero); q = 0 (ALiBi alone) and one-hot keys (forward closed forms);
//                                        v = 0 (gq = gk = 0, gv = P^T dO over all 64 dims, closed form and float
//                                        bound); head-dimension permutation equivariance across both blocks
//   para16 / para8 / soma16 (no spec) ... closed forms on exact integers (test_r16_formas_fechadas)
//   soma_est (no spec) .................. lowbias32 pinned by its published inverse; the seed layout restates
//                                        jatai_cuda.cu:375 and no vector can pin it: parity unpinned
//
// All arithmetic is int64 with two's-complement wraparound where the spec's torch int64 tensors wrap.
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <vector>
#include <immintrin.h>

typedef int64_t i64;
static const i64 E_ZERO = -127;
static const i64 SEM = -100000;

static inline i64 bitlen(i64 x) {           // ops.py:34-39
    uint64_t a = x < 0 ? (uint64_t)(-x) : (uint64_t)x;
    return a ? 64 - __builtin_clzll(a) : 0;
}
static inline i64 shl(i64 x, i64 n) { return (i64)((uint64_t)x << n); }

// x * 2^-s rounded half to even; s <= 0 is a left shift. Shift counts clamped to [0, 62] (ops.py:42-51).
static inline i64 rnd(i64 x, i64 s) {
    i64 pos = std::min<i64>(std::max<i64>(s, 0), 62), neg = std::min<i64>(std::max<i64>(-s, 0), 62);
    if (pos == 0) return shl(x, neg);
    i64 meio = (i64)1 << (pos - 1);
    i64 q = (x + meio) >> pos;
    i64 resto = x + meio - shl(q, pos);
    if (resto == 0 && (q & 1)) q -= 1;
    return q;
}

static inline i64 exp_int(i64 d) {          // exp(-d/256) in Q15 (ops.py:75-81)
    i64 t = std::min<i64>(d, 6000) * 23637;
    i64 n = t >> 22, f = (t & ((1 << 22) - 1)) >> 7;
    i64 p = -1295;
    const i64 c[3] = {7556, -22645, 32765};
    for (int i = 0; i < 3; i++) p = ((p * f) >> 15) + c[i];
    return n > 30 ? 0 : p >> std::min<i64>(n, 30);
}

static inline i64 isqrt(i64 n) {            // ops.py:84-89
    n = std::max<i64>(n, 0);
    i64 x = (i64)1 << ((bitlen(n) + 1) / 2);
    for (int i = 0; i < 10; i++) x = std::min(x, (x + n / std::max<i64>(x, 1)) >> 1);
    return std::max<i64>(x, 1);
}

static inline i64 floordiv(i64 a, i64 b) { i64 q = a / b; if ((a % b != 0) && ((a < 0) != (b < 0))) q--; return q; }
static inline int ilog2(i64 n) { int l = 0; while (((i64)2 << l) <= n) l++; return l; }   // int(math.log2(n))

// One block of `blk` values with per-element exponents -> mantissas and one exponent (ops.py:58-72).
// mbits = 7 / lim = 127 is the INT8 block format; mbits = 15 / lim = 32767 is the 16-bit residual format
// (jatai_cuda.cu:451-483, same rules with 15 bits).
template <typename MT>
static void quant_bloco(const i64* v, const i64* e, int blk, MT* m, int8_t* E, int mbits = 7, i64 lim = 127) {
    i64 topo = SEM;
    for (int k = 0; k < blk; k++) if (v[k] != 0) topo = std::max(topo, e[k] + bitlen(v[k]));
    bool zero = topo == SEM;
    i64 Eb = topo - mbits, big = 0;
    for (int k = 0; k < blk; k++) { i64 q = rnd(v[k], Eb - e[k]); big |= (q > lim || q < -lim); }
    if (big) Eb += 1;
    zero = zero || Eb < -126;
    for (int k = 0; k < blk; k++) {
        i64 q = zero ? 0 : rnd(v[k], Eb - e[k]);
        q = std::min<i64>(std::max<i64>(q, -lim), lim);
        m[k] = (MT)q;
    }
    *E = (int8_t)(zero ? E_ZERO : Eb);
}

// quant over rows of length C (C % blk == 0): v, e [R, C]
template <typename MT>
static void quant_linhas(const i64* v, const i64* e, i64 R, int C, int blk, MT* m, int8_t* E, int mbits = 7, i64 lim = 127) {
    const int nb = C / blk;
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < R; r++)
        for (int b = 0; b < nb; b++)
            quant_bloco<MT>(v + r * C + b * blk, e + r * C + b * blk, blk, m + r * C + b * blk, E + r * nb + b, mbits, lim);
}

// rnd(x, s) of 8 int32 lanes for 0 <= s and |x| < 2^26: the GEMM's per-block rounding. Every s >= 27 gives 0
// there, so s is clamped to 30, where x + 2^(s-1) still fits int32.
static inline __m256i rnd8(__m256i x, __m256i s) {
    const __m256i um = _mm256_set1_epi32(1), zero = _mm256_setzero_si256();
    s = _mm256_min_epi32(s, _mm256_set1_epi32(30));
    __m256i meio = _mm256_srli_epi32(_mm256_sllv_epi32(um, s), 1);          // 2^(s-1), 0 at s = 0
    __m256i t = _mm256_add_epi32(x, meio);
    __m256i q = _mm256_srav_epi32(t, s);
    __m256i resto = _mm256_sub_epi32(t, _mm256_sllv_epi32(q, s));
    __m256i par = _mm256_and_si256(_mm256_cmpeq_epi32(resto, zero),
                                   _mm256_and_si256(_mm256_cmpeq_epi32(_mm256_and_si256(q, um), um), _mm256_cmpgt_epi32(s, zero)));
    return _mm256_add_epi32(q, par);                                           // ties to even: q - 1 where q is odd
}

// acc[i, j] = sum_q rnd(16 * dot(A_iq, B_jq), (RA_i - ea_iq) + (RB_j - eb_jq)) for an even block size <= 128:
// the scalar loop of or_gemm, evaluated 4 rows x 16 columns at a time with 16-bit pair products (vpmaddwd).
static void gemm_acc_avx2(const int8_t* a, const int8_t* ea, const int8_t* b, const int8_t* eb, int M, int N, int K, int blk,
                          const i64* RA, const i64* RB, i64* acc) {
    const int nb = K / blk, K2 = K / 2, NT = (N + 15) / 16, MT = (M + 3) / 4, B2 = blk / 2;
    std::vector<int32_t> Ap((size_t)M * K2);                 // (a[2k], a[2k+1]) as two int16 in one int32
    std::vector<int16_t> Bp((size_t)NT * K2 * 32);           // tile t, pair k: 16 columns x (b[2k], b[2k+1])
    std::vector<int32_t> SB((size_t)NT * nb * 16);           // RB_j - eb_jq; padded columns 0
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++)
        for (int k = 0; k < K2; k++)
            Ap[(size_t)i * K2 + k] = (int32_t)(((uint32_t)(uint16_t)(int16_t)a[(i64)i * K + 2 * k]) |
                                               ((uint32_t)(uint16_t)(int16_t)a[(i64)i * K + 2 * k + 1] << 16));
#pragma omp parallel for schedule(static)
    for (int t = 0; t < NT; t++) {
        for (int k = 0; k < K2; k++)
            for (int c = 0; c < 16; c++) {
                int j = t * 16 + c;
                int16_t* d = &Bp[((size_t)t * K2 + k) * 32 + 2 * c];
                d[0] = j < N ? b[(i64)j * K + 2 * k] : 0;
                d[1] = j < N ? b[(i64)j * K + 2 * k + 1] : 0;
            }
        for (int q = 0; q < nb; q++)
            for (int c = 0; c < 16; c++) {
                int j = t * 16 + c;
                SB[((size_t)t * nb + q) * 16 + c] = j < N ? (int32_t)(RB[j] - eb[(i64)j * nb + q]) : 0;
            }
    }
#pragma omp parallel for schedule(dynamic, 1)
    for (int u = 0; u < MT; u++) {
        int rows[4];
        for (int r = 0; r < 4; r++) rows[r] = std::min(4 * u + r, M - 1);
        for (int t = 0; t < NT; t++) {
            __m256i s64[4][4];
            for (int r = 0; r < 4; r++)
                for (int h = 0; h < 4; h++) s64[r][h] = _mm256_setzero_si256();
            for (int q = 0; q < nb; q++) {
                __m256i p[4][2];
                for (int r = 0; r < 4; r++) p[r][0] = p[r][1] = _mm256_setzero_si256();
                const int16_t* bq = &Bp[((size_t)t * K2 + (size_t)q * B2) * 32];
                const int32_t* aq[4];
                for (int r = 0; r < 4; r++) aq[r] = &Ap[(size_t)rows[r] * K2 + (size_t)q * B2];
                for (int k = 0; k < B2; k++) {
                    __m256i b0 = _mm256_loadu_si256((const __m256i*)(bq + k * 32));
                    __m256i b1 = _mm256_loadu_si256((const __m256i*)(bq + k * 32 + 16));
                    for (int r = 0; r < 4; r++) {
                        __m256i av = _mm256_set1_epi32(aq[r][k]);
                        p[r][0] = _mm256_add_epi32(p[r][0], _mm256_madd_epi16(av, b0));
                        p[r][1] = _mm256_add_epi32(p[r][1], _mm256_madd_epi16(av, b1));
                    }
                }
                const int32_t* sb = &SB[((size_t)t * nb + q) * 16];
                __m256i sb0 = _mm256_loadu_si256((const __m256i*)sb), sb1 = _mm256_loadu_si256((const __m256i*)(sb + 8));
                for (int r = 0; r < 4; r++) {
                    __m256i sa = _mm256_set1_epi32((int32_t)(RA[rows[r]] - ea[(i64)rows[r] * nb + q]));
                    __m256i r0 = rnd8(_mm256_slli_epi32(p[r][0], 4), _mm256_add_epi32(sa, sb0));
                    __m256i r1 = rnd8(_mm256_slli_epi32(p[r][1], 4), _mm256_add_epi32(sa, sb1));
                    s64[r][0] = _mm256_add_epi64(s64[r][0], _mm256_cvtepi32_epi64(_mm256_castsi256_si128(r0)));
                    s64[r][1] = _mm256_add_epi64(s64[r][1], _mm256_cvtepi32_epi64(_mm256_extracti128_si256(r0, 1)));
                    s64[r][2] = _mm256_add_epi64(s64[r][2], _mm256_cvtepi32_epi64(_mm256_castsi256_si128(r1)));
                    s64[r][3] = _mm256_add_epi64(s64[r][3], _mm256_cvtepi32_epi64(_mm256_extracti128_si256(r1, 1)));
                }
            }
            for (int r = 0; r < 4; r++) {
                int i = 4 * u + r;
                if (i >= M) break;
                alignas(32) i64 o[16];
                for (int h = 0; h < 4; h++) _mm256_store_si256((__m256i*)(o + 4 * h), s64[r][h]);
                for (int c = 0; c < 16 && t * 16 + c < N; c++) acc[(i64)i * N + t * 16 + c] = o[c];
            }
        }
    }
}

extern "C" {

// ---------------------------------------------------------------- primitives (exposed for the tests)
void or_bitlen(const i64* x, i64* out, i64 n) { for (i64 i = 0; i < n; i++) out[i] = bitlen(x[i]); }
void or_rnd(const i64* x, const i64* s, i64* out, i64 n) { for (i64 i = 0; i < n; i++) out[i] = rnd(x[i], s[i]); }
void or_exp_int(const i64* d, i64* out, i64 n) { for (i64 i = 0; i < n; i++) out[i] = exp_int(d[i]); }
void or_isqrt(const i64* x, i64* out, i64 n) { for (i64 i = 0; i < n; i++) out[i] = isqrt(x[i]); }

// ---------------------------------------------------------------- quant (raw -> block), ops.py:125-126
void or_quant(const int32_t* acc, const int16_t* e, i64 R, int C, int blk, int8_t* m, int8_t* E) {
    std::vector<i64> v(R * C), ee(R * C);
    for (i64 i = 0; i < R * C; i++) { v[i] = acc[i]; ee[i] = e[i]; }
    quant_linhas<int8_t>(v.data(), ee.data(), R, C, blk, m, E);
}

// ---------------------------------------------------------------- GEMM, ops.py:95-108
// C = A . B^T, A [M,K], B [N,K] blocked along K. cru = 1: raw (acc int32, base int16); cru = 0: block output.
void or_gemm(const int8_t* a, const int8_t* ea, const int8_t* b, const int8_t* eb, int M, int N, int K, int blk, int cru,
             int8_t* cm, int8_t* cE, int32_t* c32, int16_t* ce) {
    const int nb = K / blk;
    std::vector<i64> RA(M), RB(N);
    for (int i = 0; i < M; i++) { i64 r = -1000; for (int q = 0; q < nb; q++) r = std::max<i64>(r, ea[(i64)i * nb + q]); RA[i] = r; }
    for (int j = 0; j < N; j++) { i64 r = -1000; for (int q = 0; q < nb; q++) r = std::max<i64>(r, eb[(i64)j * nb + q]); RB[j] = r; }
    std::vector<i64> acc((i64)M * N), base((i64)M * N);
    // p = exact int32 dot product of one K-block (|p| <= blk 128^2 <= 2^21), then the spec's per-block rounding
    if (blk % 2 == 0 && blk <= 128) {
        gemm_acc_avx2(a, ea, b, eb, M, N, K, blk, RA.data(), RB.data(), acc.data());
        for (int i = 0; i < M; i++)
            for (int j = 0; j < N; j++) base[(i64)i * N + j] = RA[i] + RB[j] - 4;
    } else {
#pragma omp parallel for schedule(dynamic, 4)
        for (int i = 0; i < M; i++) {
            const int8_t* ar = a + (i64)i * K;
            for (int j = 0; j < N; j++) {
                const int8_t* br = b + (i64)j * K;
                i64 s = 0;
                for (int q = 0; q < nb; q++) {
                    int32_t p = 0;
                    for (int k = 0; k < blk; k++) p += (int32_t)ar[q * blk + k] * (int32_t)br[q * blk + k];
                    s += rnd((i64)p << 4, (RA[i] - ea[(i64)i * nb + q]) + (RB[j] - eb[(i64)j * nb + q]));
                }
                acc[(i64)i * N + j] = s;
                base[(i64)i * N + j] = RA[i] + RB[j] - 4;
            }
        }
    }
    if (cru) {
        for (i64 x = 0; x < (i64)M * N; x++) { c32[x] = (int32_t)acc[x]; ce[x] = (int16_t)std::max<i64>(base[x], -30000); }
    } else {
        quant_linhas<int8_t>(acc.data(), base.data(), M, N, blk, cm, cE);
    }
}

// ---------------------------------------------------------------- element-wise family
// soma: ec = max(xE, yE) - 21 (ops.py:128-132)
void or_soma(const int8_t* xm, const int8_t* xE, const int8_t* ym, const int8_t* yE, i64 R, int C, int blk, int8_t* zm, int8_t* zE) {
    const int nb = C / blk;
    std::vector<i64> v(R * C), e(R * C);
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < R; r++)
        for (int c = 0; c < C; c++) {
            i64 x = r * C + c, w = r * nb + c / blk, ec = std::max<i64>(xE[w], yE[w]) - 21;
            v[x] = rnd(xm[x], ec - xE[w]) + rnd(ym[x], ec - yE[w]);
            e[x] = ec;
        }
    quant_linhas<int8_t>(v.data(), e.data(), R, C, blk, zm, zE);
}

// soma with the stochastic residual rounding of gemm_soma under jt_res_estocastico: no spec; restated from the
// kernel text, jatai_cuda.cu:146-159 (hash32, desloca_est, quant_grupo16<true>) and :375 (the seed of each value:
// 8 x the flat index of its lane's first value in the epilogue's 128-column tile, plus its slot in the lane).
static inline uint32_t hash32(uint32_t x) {
    x ^= x >> 16; x *= 0x7feb352dU; x ^= x >> 15; x *= 0x846ca68bU; x ^= x >> 16;
    return x;
}
static inline i64 desloca_est(i64 x, i64 s, uint32_t h) {
    if (s <= 0) return shl(x, std::min<i64>(-s, 31));
    s = std::min<i64>(s, 31);
    const i64 piso = x >> s, resto = x - shl(piso, s);
    const i64 u = (i64)(hash32(h ^ (uint32_t)x * 0x9E3779B1u) & (uint32_t)((1ull << s) - 1));
    return piso + (u < resto ? 1 : 0);
}
void or_hash32(const i64* x, i64* out, i64 n) { for (i64 i = 0; i < n; i++) out[i] = hash32((uint32_t)x[i]); }
void or_soma_est(const int8_t* xm, const int8_t* xE, const int8_t* ym, const int8_t* yE, i64 R, int C, int blk, int8_t* zm, int8_t* zE) {
    const int nb = C / blk;
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < R; r++) {
        std::vector<i64> v(blk);
        std::vector<uint32_t> h(blk);
        for (int b = 0; b < nb; b++) {
            const i64 w = r * nb + b, ex = xE[w], ey = yE[w], ec = std::max(ex, ey) - 21;
            i64 bl = 0;
            for (int k = 0; k < blk; k++) {
                const i64 x = r * C + b * blk + k;
                v[k] = rnd(xm[x], ec - ex) + rnd(ym[x], ec - ey);
                bl = std::max(bl, bitlen(v[k]));
                const i64 c = b * blk + k, col0 = c & ~(i64)127, cc = c & 127;
                h[k] = (uint32_t)(r * C + col0 + (cc & 60)) * 8u + (uint32_t)((cc & 3) + 4 * ((cc >> 6) & 1));
            }
            i64 E = ec + bl - 7;
            bool big = false;
            for (int k = 0; k < blk; k++) { const i64 q = desloca_est(v[k], bl - 7, h[k]); big |= q > 127 || q < -127; }
            const i64 s = big ? bl - 6 : bl - 7;
            if (big) E += 1;
            const bool zero = bl == 0 || E < -126;
            for (int k = 0; k < blk; k++) zm[r * C + b * blk + k] = zero ? 0 : (int8_t)desloca_est(v[k], s, h[k]);
            zE[w] = (int8_t)(zero ? E_ZERO : E);
        }
    }
}

// relu2: quant(max(m,0)^2, 2E) (ops.py:134-137)
void or_relu2(const int8_t* hm, const int8_t* hE, i64 R, int C, int blk, int8_t* am, int8_t* aE) {
    const int nb = C / blk;
    std::vector<i64> v(R * C), e(R * C);
    for (i64 r = 0; r < R; r++)
        for (int c = 0; c < C; c++) {
            i64 x = r * C + c, h = std::max<i64>(hm[x], 0);
            v[x] = h * h; e[x] = 2 * (i64)hE[r * nb + c / blk];
        }
    quant_linhas<int8_t>(v.data(), e.data(), R, C, blk, am, aE);
}

// relu2_back: quant(g * max(h,0) * 2, gE + hE) (ops.py:139-141)
void or_relu2_back(const int8_t* gm, const int8_t* gE, const int8_t* hm, const int8_t* hE, i64 R, int C, int blk, int8_t* om, int8_t* oE) {
    const int nb = C / blk;
    std::vector<i64> v(R * C), e(R * C);
    for (i64 r = 0; r < R; r++)
        for (int c = 0; c < C; c++) {
            i64 x = r * C + c, w = r * nb + c / blk;
            v[x] = (i64)gm[x] * std::max<i64>(hm[x], 0) * 2; e[x] = (i64)gE[w] + hE[w];
        }
    quant_linhas<int8_t>(v.data(), e.data(), R, C, blk, om, oE);
}

// transpoe: quant(m^T, expande(E)^T) (ops.py:121-123). X [R,C] -> Y [C,R]
void or_transpoe(const int8_t* xm, const int8_t* xE, int R, int C, int blk, int8_t* ym, int8_t* yE) {
    const int nbx = C / blk, nby = R / blk;
    // output row c, block b gathers column c of source rows b*blk .. b*blk+blk-1 with their own exponents;
    // 64 output rows at a time, so each source row contributes one contiguous 64-byte run
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < nby; b++)
        for (int c0 = 0; c0 < C; c0 += 64) {
            std::vector<i64> v(blk), e(blk);
            for (int c = c0; c < std::min(C, c0 + 64); c++) {
                for (int k = 0; k < blk; k++) {
                    i64 r = (i64)b * blk + k;
                    v[k] = xm[r * C + c];
                    e[k] = xE[r * nbx + c / blk];
                }
                quant_bloco<int8_t>(v.data(), e.data(), blk, ym + (i64)c * R + (i64)b * blk, yE + (i64)c * nby + b);
            }
        }
}

// embed: row gather (ops.py:143-145). Returns the number of out-of-vocabulary tokens (their rows are zeroed).
int or_embed(const int8_t* wm, const int8_t* wE, const int32_t* tok, int M, int D, int V, int blk, int8_t* xm, int8_t* xE) {
    const int nb = D / blk;
    int bad = 0;
    for (int t = 0; t < M; t++) {
        int v = tok[t];
        if (v < 0 || v >= V) {
            bad++;
            memset(xm + (i64)t * D, 0, D); memset(xE + (i64)t * nb, (int8_t)E_ZERO, nb);
            continue;
        }
        memcpy(xm + (i64)t * D, wm + (i64)v * D, D);
        memcpy(xE + (i64)t * nb, wE + (i64)v * nb, nb);
    }
    return bad;
}

// um_quente: one-hot int8 rows, exponent 0 (ops.py:147-151)
int or_um_quente(const int32_t* tok, int M, int V, int blk, int8_t* U, int8_t* UE) {
    int bad = 0;
    memset(U, 0, (size_t)M * V);
    memset(UE, 0, (size_t)M * (V / blk));
    for (int t = 0; t < M; t++) {
        if (tok[t] < 0 || tok[t] >= V) { bad++; continue; }
        U[(i64)t * V + tok[t]] = 1;
    }
    return bad;
}

// (G of the RMSNorm, G of its backward) = g_rms(D) (ops.py:28-30)
void or_g_rms(int D, int blk, int* G, int* GB) {
    int nb = D / blk;
    *G = 2 * (int)floordiv(8 - ilog2(nb), 2);
    *GB = 14 - ilog2(D);
}

// rms (ops.py:153-165): Y block [M,D], r and emax int32 [M]
void or_rms(const int8_t* xm, const int8_t* xE, int M, int D, int blk, int8_t* ym, int8_t* yE, int32_t* cr, int32_t* cemax) {
    const int nb = D / blk, lg = ilog2(D);
    int G, GB;
    or_g_rms(D, blk, &G, &GB);
    std::vector<i64> v((i64)M * D), e((i64)M * D);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++) {
        const int8_t* x = xm + (i64)i * D;
        i64 emax = -1000;
        for (int b = 0; b < nb; b++) emax = std::max<i64>(emax, xE[(i64)i * nb + b]);
        i64 ss = 0;
        for (int b = 0; b < nb; b++) {
            i64 sq = 0;
            for (int k = 0; k < blk; k++) sq += (i64)x[b * blk + k] * x[b * blk + k];
            ss += rnd(sq << G, 2 * (emax - xE[(i64)i * nb + b]));
        }
        i64 r = isqrt(ss >> lg), k = bitlen(r) + 10, inv = ((i64)1 << k) / r;
        for (int c = 0; c < D; c++) {
            v[(i64)i * D + c] = (i64)x[c] * inv;
            e[(i64)i * D + c] = (i64)xE[(i64)i * nb + c / blk] - k - emax + G / 2;
        }
        cr[i] = (int32_t)r; cemax[i] = (int32_t)emax;
    }
    quant_linhas<int8_t>(v.data(), e.data(), M, D, blk, ym, yE);
}

// rms_back (ops.py:167-184)
void or_rms_back(const int8_t* gm, const int8_t* gE, const int8_t* ym, const int8_t* yE, const int32_t* cr, const int32_t* cemax,
                 int M, int D, int blk, int8_t* om, int8_t* oE) {
    const int nb = D / blk, lg = ilog2(D);
    int G, GB;
    or_g_rms(D, blk, &G, &GB);
    std::vector<i64> v((i64)M * D), e((i64)M * D);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++) {
        const int8_t* g = gm + (i64)i * D;
        const int8_t* y = ym + (i64)i * D;
        const int8_t* ge = gE + (i64)i * nb;
        const int8_t* ye = yE + (i64)i * nb;
        i64 smax = -100000;
        for (int b = 0; b < nb; b++) smax = std::max<i64>(smax, (i64)ge[b] + ye[b]);
        i64 S = 0;
        for (int c = 0; c < D; c++) S += rnd(((i64)g[c] * y[c]) << GB, smax - ((i64)ge[c / blk] + ye[c / blk]));
        i64 eS = smax - GB - lg;
        i64 sh = std::max<i64>(bitlen(S) - 15, 0);
        S = rnd(S, sh); eS += sh;
        i64 r = cr[i], emax = cemax[i], k = bitlen(r) + 10, inv = ((i64)1 << k) / r;
        for (int c = 0; c < D; c++) {
            i64 egb = ge[c / blk], eyb = ye[c / blk];
            i64 ec = std::max<i64>(egb + 7, eyb + eS + 22) - 28;
            i64 dentro = rnd(g[c], ec - egb) - rnd((i64)y[c] * S, ec - (eyb + eS));
            i64 sh2 = std::max<i64>(bitlen(dentro) - 18, 0);
            dentro = rnd(dentro, sh2);
            v[(i64)i * D + c] = dentro * inv;
            e[(i64)i * D + c] = ec + sh2 - k - (emax - G / 2);
        }
    }
    quant_linhas<int8_t>(v.data(), e.data(), M, D, blk, om, oE);
}

// ---------------------------------------------------------------- attention (ops.py:186-258)
// Heads of width hd = D / H. The spec fixes hd = 4 (ops.py:188,196); the general form below is this build's
// declared extension and reduces to the spec at hd = 4:
//   alignment: every value of head h in token t is aligned to emx = the largest block exponent the head spans
//              over all T tokens of its sequence (at hd = 4 a head spans one block);
//   score:     u = rnd(q.k, -(eq + ek - log2(hd)/2 + 8))   (the spec's -1 is -log2(4)/2);
//   ALiBi:     incl = 8 - h // 8 at hd = 4 for every H (the spec, ops.py:208); for hd > 4, incl = 8 - (8 h) / H
//              (eight slopes 2^0 .. 2^-7 spread evenly over the H heads; at H = 64 the same as the spec's);
//   dS:        shrunk to 12 - max(0, ceil(log2 T) - 7) bits (12 for T <= 128, keeping |gq|,|gk| < 2^30).
static int att_lg(int hd) { return ilog2(hd) / 2; }
static int att_dsbits(int T) { return 12 - std::max(0, ilog2(2 * T - 1) - 7); }
int or_att_dsbits(int T) { return att_dsbits(T); }
static i64 att_incl(int h, int H, int hd) { return hd == 4 ? 8 - h / 8 : 8 - (8 * (i64)h) / H; }

// aligned values a[t][d] = rnd(x << GA, emx - e) and the head exponent emx - GA (ops.py:186-192)
static void alinha(const int8_t* m, const int8_t* E, int ld, int col0, int blk, int b, int T, int hd, int GA,
                   std::vector<i64>& a, i64& eo) {
    const int nbl = ld / blk;
    i64 emx = -100000;
    for (int t = 0; t < T; t++)
        for (int d = 0; d < hd; d += 1) emx = std::max<i64>(emx, E[(i64)(b * T + t) * nbl + (col0 + d) / blk]);
    a.assign((size_t)T * hd, 0);
    for (int t = 0; t < T; t++)
        for (int d = 0; d < hd; d++) {
            i64 e = E[(i64)(b * T + t) * nbl + (col0 + d) / blk];
            a[(size_t)t * hd + d] = rnd((i64)m[(i64)(b * T + t) * ld + col0 + d] << GA, emx - e);
        }
    eo = emx - GA;
}

// qkv block [Bt*T, 3D] -> oacc int32 [Bt*T, D], oe int16 [Bt*T, D], P uint8 [Bt*H, T(j), T(i)] (stored transposed)
void or_atencao(const int8_t* qm, const int8_t* qE, int Bt, int T, int H, int D, int blk, int GA,
                int32_t* oacc, int16_t* oe, uint8_t* P) {
    const int hd = D / H, ld = 3 * D, lg = att_lg(hd);
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < Bt * H; bh++) {
        const int b = bh / H, h = bh % H;
        std::vector<i64> qa, ka, va;
        i64 eq, ek, ev;
        alinha(qm, qE, ld, h * hd, blk, b, T, hd, GA, qa, eq);
        alinha(qm, qE, ld, D + h * hd, blk, b, T, hd, GA, ka, ek);
        alinha(qm, qE, ld, 2 * D + h * hd, blk, b, T, hd, GA, va, ev);
        const i64 incl = att_incl(h, H, hd), su = -(eq + ek - lg + 8);
        std::vector<i64> u(T), ex(T);
        for (int i = 0; i < T; i++) {
            i64 mx = -((i64)1 << 62);
            for (int j = 0; j <= i; j++) {
                i64 s = 0;
                for (int d = 0; d < hd; d++) s += qa[(size_t)i * hd + d] * ka[(size_t)j * hd + d];
                // the spec shifts by torch's bitwise_left_shift, which gives 0 for a negative count (incl < 0)
                u[j] = rnd(s, su) - (incl >= 0 ? shl((i64)(i - j), incl) : 0);
                mx = std::max(mx, u[j]);
            }
            i64 sum = 0;
            for (int j = 0; j <= i; j++) { ex[j] = exp_int(mx - u[j]) >> 3; sum += ex[j]; }
            i64 inv = ((i64)1 << 28) / sum;
            std::vector<i64> o(hd, 0);
            for (int j = 0; j < T; j++) {
                i64 p = 0;
                if (j <= i) {
                    p = std::min<i64>((ex[j] * inv + (1 << 19)) >> 20, 255);
                    for (int d = 0; d < hd; d++) o[d] += p * va[(size_t)j * hd + d];
                }
                P[(i64)bh * T * T + (i64)j * T + i] = (uint8_t)p;
            }
            for (int d = 0; d < hd; d++) {
                i64 x = (i64)(b * T + i) * D + h * hd + d;
                oacc[x] = (int32_t)o[d];
                oe[x] = (int16_t)(ev - 8);
            }
        }
    }
}

// go block [Bt*T, D], qkv block [Bt*T, 3D], P as written by or_atencao -> raw (acc int32, e int16) [Bt*T, 3D]
void or_atencao_back(const int8_t* gm, const int8_t* gE, const int8_t* qm, const int8_t* qE, const uint8_t* P,
                     int Bt, int T, int H, int D, int blk, int GA, int limite, int32_t* gacc, int16_t* ge) {
    const int hd = D / H, ld = 3 * D, dsb = att_dsbits(T);
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < Bt * H; bh++) {
        const int b = bh / H, h = bh % H;
        std::vector<i64> goa, qa, ka, va;
        i64 ego, eq, ek, ev;
        alinha(gm, gE, D, h * hd, blk, b, T, hd, GA, goa, ego);
        alinha(qm, qE, ld, h * hd, blk, b, T, hd, GA, qa, eq);
        alinha(qm, qE, ld, D + h * hd, blk, b, T, hd, GA, ka, ek);
        alinha(qm, qE, ld, 2 * D + h * hd, blk, b, T, hd, GA, va, ev);
        const uint8_t* Pb = P + (i64)bh * T * T;
        auto Pl = [&](int i, int j) -> i64 { return Pb[(i64)j * T + i]; };   // P[i][j]
        std::vector<i64> gP((size_t)T * T);
        for (int i = 0; i < T; i++)
            for (int j = 0; j < T; j++) {
                i64 s = 0;
                for (int d = 0; d < hd; d++) s += goa[(size_t)i * hd + d] * va[(size_t)j * hd + d];
                gP[(size_t)i * T + j] = s;
            }
        i64 sh;
        if (limite) {      // |gP_ij| <= max_i ||dO_i||_inf * max_j ||v_j||_1 (ops.py:231-233)
            i64 a1 = 0, a2 = 0;
            for (int t = 0; t < T; t++) {
                i64 s1 = 0;
                for (int d = 0; d < hd; d++) { a1 = std::max<i64>(a1, std::llabs(goa[(size_t)t * hd + d])); s1 += std::llabs(va[(size_t)t * hd + d]); }
                a2 = std::max(a2, s1);
            }
            sh = std::max<i64>(bitlen(a1 * a2) - 15, 0);
        } else {           // causal max (ops.py:235)
            i64 mg = 0;
            for (int i = 0; i < T; i++) for (int j = 0; j <= i; j++) mg = std::max<i64>(mg, std::llabs(gP[(size_t)i * T + j]));
            sh = std::max<i64>(bitlen(mg) - 15, 0);
        }
        for (auto& x : gP) x = rnd(x, sh);
        const i64 egp = ego + ev + sh;
        std::vector<i64> sl(T);
        for (int i = 0; i < T; i++) {
            i64 s = 0;
            for (int j = 0; j < T; j++) s += Pl(i, j) * gP[(size_t)i * T + j];
            sl[i] = rnd(s, 8);
        }
        std::vector<i64> dS((size_t)T * T);
        for (int i = 0; i < T; i++) for (int j = 0; j < T; j++) dS[(size_t)i * T + j] = Pl(i, j) * (gP[(size_t)i * T + j] - sl[i]);
        i64 sh2;
        if (limite) {      // max P * (causal max |gP| + max |s_lin|) (ops.py:240-242)
            i64 pm = 0, gmx = 0, sm = 0;
            for (int i = 0; i < T; i++) {
                for (int j = 0; j < T; j++) pm = std::max(pm, Pl(i, j));
                for (int j = 0; j <= i; j++) gmx = std::max<i64>(gmx, std::llabs(gP[(size_t)i * T + j]));
                sm = std::max<i64>(sm, std::llabs(sl[i]));
            }
            sh2 = std::max<i64>(bitlen(pm * (gmx + sm)) - dsb, 0);
        } else {
            i64 md = 0;
            for (auto x : dS) md = std::max<i64>(md, std::llabs(x));
            sh2 = std::max<i64>(bitlen(md) - dsb, 0);
        }
        for (auto& x : dS) x = rnd(x, sh2);
        const i64 eds = egp - 9 + sh2;
        for (int i = 0; i < T; i++) {
            const i64 row = (i64)(b * T + i) * ld;
            for (int d = 0; d < hd; d++) {
                i64 gq = 0, gk = 0, gv = 0;
                for (int j = 0; j < T; j++) {
                    gq += dS[(size_t)i * T + j] * ka[(size_t)j * hd + d];
                    gk += dS[(size_t)j * T + i] * qa[(size_t)j * hd + d];
                    gv += Pl(j, i) * goa[(size_t)j * hd + d];
                }
                const i64 c = h * hd + d;
                gacc[row + c] = (int32_t)gq;          ge[row + c] = (int16_t)(eds + ek);
                gacc[row + D + c] = (int32_t)gk;      ge[row + D + c] = (int16_t)(eds + eq);
                gacc[row + 2 * D + c] = (int32_t)gv;  ge[row + 2 * D + c] = (int16_t)(ego - 8);
            }
        }
    }
}

// ---------------------------------------------------------------- softmax cross-entropy (ops.py:260-271)
// Returns the number of out-of-range targets (those rows are skipped).
int or_softmax_ce(const int32_t* acc, const int16_t* e, const int32_t* alvo, int M, int V, int blk,
                  int8_t* gm, int8_t* gE, int32_t* d_alvo, int32_t* soma) {
    const int lgM = ilog2(M);
    std::vector<i64> v((i64)M * V), ee((i64)M * V, -12 - lgM);
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (int i = 0; i < M; i++) {
        std::vector<i64> u(V);
        i64 umax = INT64_MIN;
        for (int c = 0; c < V; c++) { u[c] = rnd(acc[(i64)i * V + c], -((i64)e[(i64)i * V + c] + 8)); umax = std::max(umax, u[c]); }
        i64 s = 0;
        std::vector<i64> ex(V);
        for (int c = 0; c < V; c++) { ex[c] = exp_int(umax - u[c]) >> 3; s += ex[c]; }
        i64 inv = ((i64)1 << 28) / s;
        for (int c = 0; c < V; c++) v[(i64)i * V + c] = (ex[c] * inv + (1 << 15)) >> 16;
        const int t = alvo[i];
        if (t < 0 || t >= V) { bad++; d_alvo[i] = 0; soma[i] = (int32_t)s; continue; }
        v[(i64)i * V + t] -= 4096;
        d_alvo[i] = (int32_t)(umax - u[t]);
        soma[i] = (int32_t)s;
    }
    quant_linhas<int8_t>(v.data(), ee.data(), M, V, blk, gm, gE);
    return bad;
}

// ---------------------------------------------------------------- optimizer
// momento: Mom <- 7/8 Mom + g, in place (ops.py:273-278). n = number of elements.
void or_momento(const int32_t* g, const int16_t* ge, int8_t* mm, int8_t* mE, i64 n, int blk) {
    std::vector<i64> v(n), e(n);
    for (i64 x = 0; x < n; x++) {
        i64 em = (i64)mE[x / blk] - 3;
        i64 ec = std::max<i64>(em + 10, (i64)ge[x] + bitlen(g[x])) - 28;
        v[x] = rnd((i64)mm[x] * 7, ec - em) + rnd(g[x], ec - ge[x]);
        e[x] = ec;
    }
    quant_linhas<int8_t>(v.data(), e.data(), n / blk, blk, blk, mm, mE);
}

// peso: W <- W - 2^-k Mom (+ error-feedback residual R), in place (ops.py:280-290)
void or_peso(int8_t* wm, int8_t* wE, const int8_t* mm, const int8_t* mE, int8_t* rm, int8_t* rE, int k, int ef, i64 n, int blk) {
    std::vector<i64> alvo(n), e(n);
    for (i64 x = 0; x < n; x++) {
        i64 w = x / blk, ew = wE[w], em = (i64)mE[w] - k, er = ef ? (i64)rE[w] : E_ZERO;
        i64 ec = std::max(std::max(ew + 7, em + 7), er + 7) - 27;
        alvo[x] = rnd(wm[x], ec - ew) - rnd(mm[x], ec - em) + (ef ? rnd(rm[x], ec - er) : 0);
        e[x] = ec;
    }
    quant_linhas<int8_t>(alvo.data(), e.data(), n / blk, blk, blk, wm, wE);
    if (!ef) return;
    std::vector<i64> dif(n);
    for (i64 x = 0; x < n; x++) dif[x] = alvo[x] - (wm[x] == 0 ? 0 : rnd(wm[x], e[x] - (i64)wE[x / blk]));
    quant_linhas<int8_t>(dif.data(), e.data(), n / blk, blk, blk, rm, rE);
}

// ---------------------------------------------------------------- 16-bit residual stream (jatai_cuda.cu:446-531)
// para16: INT8 -> R16, exact (m << 7, E - 7; zero blocks keep E = -127)
void or_para16(const int8_t* xm, const int8_t* xE, i64 n, int blk, int16_t* zm, int8_t* zE) {
    for (i64 x = 0; x < n; x++) zm[x] = (int16_t)((int)xm[x] << 7);
    for (i64 w = 0; w < n / blk; w++) zE[w] = xE[w] == E_ZERO ? (int8_t)E_ZERO : (int8_t)(xE[w] - 7);
}
// para8: R16 -> INT8 with the INT8 quant rules
void or_para8(const int16_t* xm, const int8_t* xE, i64 n, int blk, int8_t* ym, int8_t* yE) {
    std::vector<i64> v(n), e(n);
    for (i64 x = 0; x < n; x++) { v[x] = xm[x]; e[x] = xE[x / blk]; }
    quant_linhas<int8_t>(v.data(), e.data(), n / blk, blk, blk, ym, yE);
}
// soma16: R16 + INT8 -> R16, ec = max(ex + 15, ey + 7) - 28, zero blocks contribute 0
void or_soma16(const int16_t* xm, const int8_t* xE, const int8_t* ym, const int8_t* yE, i64 n, int blk, int16_t* zm, int8_t* zE) {
    std::vector<i64> v(n), e(n);
    for (i64 x = 0; x < n; x++) {
        i64 w = x / blk, ex = xE[w], ey = yE[w], ec = std::max(ex + 15, ey + 7) - 28;
        v[x] = (ex == E_ZERO ? 0 : rnd(xm[x], ec - ex)) + (ey == E_ZERO ? 0 : rnd(ym[x], ec - ey));
        e[x] = ec;
    }
    quant_linhas<int16_t>(v.data(), e.data(), n / blk, blk, blk, zm, zE, 15, 32767);
}

}  // extern "C"
