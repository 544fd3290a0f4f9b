/* sincos_check.c - CPU restatement of the device rot_of (getting-over-it-rl_amd/csrc/b2_math.hpp) in the same double
 * operations, checked against the oracle's definition (float)sin((double)x), (float)cos((double)x) of the C library.
 *
 *   sincos_check LO HI [STRIDE]   every STRIDE-th float bit pattern u in [LO, HI) (|x| < 2^20: the table path;
 *                                 larger angles take the library itself on the device)
 *   -DPLANT_FACTORED              builds a planted mistake (the factored addition formulas) for the test's check
 *
 * Prints the number checked and the mismatches (the first few with their inputs); exit status 1 on any mismatch.
 * Built with -ffp-contract=off so that no operation fuses beyond the fma() calls written here.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../getting-over-it-rl_amd/csrc/b2_sincos_table.h"

static const double kTable[128] = {GOI_SINCOS_TABLE};

static void table_sincos(float a, float* so, float* co) {
    const double x = (double)a;
    const double k = rint(x * GOI_SC_32_OVER_PI);
    double r = fma(-k, GOI_SC_P1, x);
    r = fma(-k, GOI_SC_P2, r);
    r = fma(-k, GOI_SC_P3, r);
    const double r2 = r * r;
    double ps = GOI_SC_S9;
    ps = fma(ps, r2, GOI_SC_S7);
    ps = fma(ps, r2, GOI_SC_S5);
    ps = fma(ps, r2, GOI_SC_S3);
    double pc = GOI_SC_C8;
    pc = fma(pc, r2, GOI_SC_C6);
    pc = fma(pc, r2, GOI_SC_C4);
    pc = fma(pc, r2, GOI_SC_C2);
    const double sr = fma(r * r2, ps, r), cm1 = r2 * pc;
    const int j = (int)k & 63;
    const double st = kTable[2 * j], ct = kTable[2 * j + 1];
#ifdef PLANT_FACTORED /* a planted mistake: the factored addition formulas, sin x = St cos r + Ct sin r */
    const double cr = fma(r2, pc, 1.0);
    const double s = fma(st, cr, ct * sr);
    const double c = fma(ct, cr, -(st * sr));
#else
    const double s = st + fma(st, cm1, ct * sr);
    const double c = ct + fma(ct, cm1, -(st * sr));
#endif
    *so = a == 0.0f ? a : (float)s;
    *co = (float)c;
}

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    const int64_t lo = (int64_t)strtoull(argv[1], 0, 0), hi = (int64_t)strtoull(argv[2], 0, 0);
    const int64_t stride = argc > 3 ? (int64_t)strtoull(argv[3], 0, 0) : 1;
    long n = 0, bad = 0;
#pragma omp parallel for reduction(+ : n, bad) schedule(dynamic, 1)
    for (int64_t b0 = lo; b0 < hi; b0 += stride << 16) {
        const int64_t b1 = b0 + (stride << 16) < hi ? b0 + (stride << 16) : hi;
        for (int64_t u = b0; u < b1; u += stride) {
            const uint32_t bits = (uint32_t)u;
            float x, s, c;
            memcpy(&x, &bits, 4);
            table_sincos(x, &s, &c);
            const float rs = (float)sin((double)x), rc = (float)cos((double)x);
            if (memcmp(&s, &rs, 4) || memcmp(&c, &rc, 4)) {
                if (bad < 8) printf("mismatch x=%a: sin %a vs %a, cos %a vs %a\n", x, s, rs, c, rc);
                ++bad;
            }
            ++n;
        }
    }
    printf("checked %ld mismatches %ld\n", n, bad);
    return bad != 0;
}
