/*
 * CPU oracle for the EXL3 trellis linear path.  TEST INFRASTRUCTURE ONLY: this file is
 * the checker that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * compare the HIP library against.  Nothing in the product links or calls it.
 *
 * What it restates (reference = jschang/OrcaSAQ2-kernel, read as text):
 *   - trellis shape (ic/16, oc/16, 16K) int16 and K = last_dim/16 ...... orcasaq2/ops.py:28-34
 *   - reconstruct: W_q (ic, oc) fp16 row-major from the trellis ........ orcasaq2/ops.py:55-56,
 *                                                                         orcasaq2/__init__.py:53-57
 *   - codebook flags: mcg / mul1 from the presence of tensors .......... orcasaq2/config.py:218
 * The trellis arithmetic itself lives in exllamav3 v1.5.1 (absent from the reference
 * tree), so the decode below follows the published QTIP method (arXiv 2406.11235,
 * "bitshift trellis" + "3INST" codebook) with the layout choices written out here:
 *
 *   Stream.  A tile's 16K int16 words are read as 8K little-endian u32 words
 *     u[j] = w[2j] | w[2j+1] << 16.  Stream bit p (0 <= p < 256K) is bit 31 - p%32 of
 *     u[p/32] (MSB-first within each 32-bit word).
 *   State.   Position t (0..255) has the 16-bit state formed by stream bits
 *     [(t+1)K - 16, (t+1)K) taken modulo 256K (tail-biting), earliest bit most
 *     significant.  So the K newest bits of a step are the state's low bits and
 *     s_{t+1} >> K == s_t & (2^(16-K) - 1).
 *   Placement.  Position t = 8j + i (j = 0..31, i = 0..7) lands at tile row
 *     2(j%4) + {0,1,8,9}[i%4] and tile column j/4 + 8(i/4) (16x16 MMA-fragment order);
 *     tile (ti, tn) covers W_q rows 16ti.. and columns 16tn..
 *   3INST.   x = (89226354 s + 64248484) mod 2^32; x = (x & 0x8FFF8FFF) ^ 0x3B603B60;
 *     value = fp16(lo16(x)) + fp16(hi16(x)) with one IEEE round-to-nearest-even.
 *   MCG.     x = (0xCBAC1FED s) mod 2^32, then the same mask / xor / half-sum.
 *
 * Parity with exllamav3's own bit order, placement and MCG multiplier is unpinned (the
 * extension is absent); tests pin this file against the codebook statistics of the
 * published constants, the shift-register property of a tail-biting trellis,
 * hand-computed known answers and brute force.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------- fp16 <-> fp32/fp64, IEEE binary16, round to nearest even ---------------- */

float exl3o_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                                   /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Correctly rounded double -> binary16 (one rounding, ties to even). */
uint16_t exl3o_double_to_half(double d)
{
    uint16_t sign = signbit(d) ? 0x8000 : 0;
    double a = fabs(d);
    if (isnan(d)) return 0x7e00;
    if (a >= 65520.0) return sign | 0x7c00;       /* rounds to inf */
    if (a < 5.9604644775390625e-08 / 2)           /* below half the smallest subnormal */
        return sign;
    int e;
    frexp(a, &e);                                 /* a = m * 2^e, m in [0.5, 1) */
    int exp_unb = e - 1;                          /* a in [2^exp_unb, 2^(exp_unb+1)) */
    double q;                                     /* quantum (ulp) at this magnitude */
    if (exp_unb < -14) q = ldexp(1.0, -24);
    else q = ldexp(1.0, exp_unb - 10);
    double n = a / q;                             /* exact: power-of-two scaling */
    double fl = floor(n);
    double rem = n - fl;
    if (rem > 0.5 || (rem == 0.5 && fmod(fl, 2.0) != 0.0)) fl += 1.0;
    double r = fl * q;
    /* re-encode r (exact in binary16 by construction) */
    if (r == 0.0) return sign;
    int e2;
    frexp(r, &e2);
    int eu = e2 - 1;
    if (eu < -14) {
        return sign | (uint16_t)(r / ldexp(1.0, -24));
    }
    if (eu > 15) return sign | 0x7c00;
    uint32_t man = (uint32_t)(r / ldexp(1.0, eu - 10)) - 1024u;
    return sign | (uint16_t)(((eu + 15) << 10) | man);
}

uint16_t exl3o_float_to_half(float f) { return exl3o_double_to_half((double)f); }

/* ---------------- trellis stream, state window, placement ---------------- */

static inline uint32_t stream_bit(const uint16_t *tile, int K, long p)
{
    long nbits = 256L * K;
    p %= nbits;
    if (p < 0) p += nbits;
    long j = p >> 5;
    uint32_t u = (uint32_t)tile[2 * j] | ((uint32_t)tile[2 * j + 1] << 16);
    return (u >> (31 - (p & 31))) & 1u;
}

/* 16-bit state of position t of one tile (16K words). */
uint32_t exl3o_state(const uint16_t *tile, int K, int t)
{
    long start = (long)(t + 1) * K - 16;
    uint32_t s = 0;
    for (int i = 0; i < 16; i++) s = (s << 1) | stream_bit(tile, K, start + i);
    return s;
}

/* Tile-local placement of position t: returns row * 16 + col. */
int exl3o_perm(int t)
{
    static const int roff[4] = {0, 1, 8, 9};
    int j = t >> 3, i = t & 7;
    int row = 2 * (j & 3) + roff[i & 3];
    int col = (j >> 2) + 8 * (i >> 2);
    return row * 16 + col;
}

/* ---------------- codebooks ---------------- */

enum { EXL3O_CB_3INST = 0, EXL3O_CB_MCG = 1 };

/* fp16 bits of the codebook value of a 16-bit state. */
uint16_t exl3o_codebook(uint32_t s, int cb)
{
    uint32_t x;
    s &= 0xffffu;
    if (cb == EXL3O_CB_MCG) x = s * 0xCBAC1FEDu;
    else x = s * 89226354u + 64248484u;
    x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    double lo = exl3o_half_to_float((uint16_t)(x & 0xffffu));
    double hi = exl3o_half_to_float((uint16_t)(x >> 16));
    return exl3o_double_to_half(lo + hi);          /* exact sum, one rounding */
}

/* Whole 2^16-entry table (fp16 bits), for fixtures and statistics. */
void exl3o_codebook_table(uint16_t *out, int cb)
{
    for (uint32_t s = 0; s < 65536u; s++) out[s] = exl3o_codebook(s, cb);
}

/* Decode one tile to a 16x16 row-major fp16 block. */
void exl3o_decode_tile(uint16_t *out256, const uint16_t *tile, int K, int cb)
{
    for (int t = 0; t < 256; t++) out256[exl3o_perm(t)] = exl3o_codebook(exl3o_state(tile, K, t), cb);
}

/* W_q (ic, oc) fp16 row-major from trellis (ic/16, oc/16, 16K). */
void exl3o_reconstruct(uint16_t *W, const uint16_t *trellis, int ic, int oc, int K, int cb,
                       int nthreads)
{
    int tr = ic / 16, tc = oc / 16;
    long tiles = (long)tr * tc;
    int words = 16 * K;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (long tidx = 0; tidx < tiles; tidx++) {
        int ti = (int)(tidx / tc), tn = (int)(tidx % tc);
        const uint16_t *tile = trellis + tidx * words;
        uint16_t blk[256];
        exl3o_decode_tile(blk, tile, K, cb);
        for (int r = 0; r < 16; r++)
            memcpy(W + (long)(16 * ti + r) * oc + 16 * tn, blk + 16 * r, 32);
    }
}

/* ---------------- block-128 Walsh-Hadamard (fp64) ---------------- */

/* In place, rows x cols (cols % 128 == 0): every 128-block of a row times H128/sqrt(128),
 * H128 the Sylvester matrix ([[h, h], [h, -h]] doubling) as in orcasaq2/__init__.py:33-46. */
void exl3o_had128(double *x, long rows, int cols)
{
    const double norm = 1.0 / sqrt(128.0);
    for (long r = 0; r < rows; r++) {
        for (int b = 0; b < cols; b += 128) {
            double *v = x + r * cols + b;
            for (int h = 1; h < 128; h <<= 1)
                for (int i = 0; i < 128; i += 2 * h)
                    for (int j = i; j < i + h; j++) {
                        double a = v[j], c = v[j + h];
                        v[j] = a + c;
                        v[j + h] = a - c;
                    }
            for (int j = 0; j < 128; j++) v[j] *= norm;
        }
    }
}
