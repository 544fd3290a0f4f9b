/* b2_sincos_table.h - the constants of rot_of's float sin/cos (b2_math.hpp), plain C so that the device code and
 * its CPU checker (tests/sincos_check.c) read the same numbers.
 *
 * x = k pi/32 + r with k = rint(x * 32/pi) and pi/32 = P1 + P2 + P3 (each the nearest double to what remains of pi/32),
 * r by three fused multiply-adds; |r| <= pi/64 + tiny.
 * sin r = r + r^3 (S3 + r^2 (S5 + r^2 (S7 + r^2 S9))), cos r - 1 = r^2 (C2 + r^2 (C4 + r^2 (C6 + r^2 C8))): the
 * Taylor coefficients (-1)^n/(2n+1)! and (-1)^n/(2n)!, truncation below 2^-65 relative on |r| <= pi/64.
 * GOI_SINCOS_TABLE: for j = 0..63 the doubles nearest to sin(j pi/32) and cos(j pi/32) (exact zeros and +-1 at the
 * multiples of pi/2).
 * Generated with 400-bit mpmath arithmetic.
 */
#ifndef GOI_B2_SINCOS_TABLE_H
#define GOI_B2_SINCOS_TABLE_H

#define GOI_SC_32_OVER_PI 0x1.45f306dc9c883p+3
#define GOI_SC_P1 0x1.921fb54442d18p-4
#define GOI_SC_P2 0x1.1a62633145c07p-58
#define GOI_SC_P3 -0x1.f1976b7ed8fbcp-114
#define GOI_SC_S3 -0x1.5555555555555p-3
#define GOI_SC_S5 0x1.1111111111111p-7
#define GOI_SC_S7 -0x1.a01a01a01a01ap-13
#define GOI_SC_S9 0x1.71de3a556c734p-19
#define GOI_SC_C2 -0x1.0000000000000p-1
#define GOI_SC_C4 0x1.5555555555555p-5
#define GOI_SC_C6 -0x1.6c16c16c16c17p-10
#define GOI_SC_C8 0x1.a01a01a01a01ap-16

#define GOI_SINCOS_TABLE \
    0x0.0p+0, 0x1.0000000000000p+0, \
    0x1.917a6bc29b42cp-4, 0x1.fd88da3d12526p-1, \
    0x1.8f8b83c69a60bp-3, 0x1.f6297cff75cb0p-1, \
    0x1.294062ed59f06p-2, 0x1.e9f4156c62ddap-1, \
    0x1.87de2a6aea963p-2, 0x1.d906bcf328d46p-1, \
    0x1.e2b5d3806f63bp-2, 0x1.c38b2f180bdb1p-1, \
    0x1.1c73b39ae68c8p-1, 0x1.a9b66290ea1a3p-1, \
    0x1.44cf325091dd6p-1, 0x1.8bc806b151741p-1, \
    0x1.6a09e667f3bcdp-1, 0x1.6a09e667f3bcdp-1, \
    0x1.8bc806b151741p-1, 0x1.44cf325091dd6p-1, \
    0x1.a9b66290ea1a3p-1, 0x1.1c73b39ae68c8p-1, \
    0x1.c38b2f180bdb1p-1, 0x1.e2b5d3806f63bp-2, \
    0x1.d906bcf328d46p-1, 0x1.87de2a6aea963p-2, \
    0x1.e9f4156c62ddap-1, 0x1.294062ed59f06p-2, \
    0x1.f6297cff75cb0p-1, 0x1.8f8b83c69a60bp-3, \
    0x1.fd88da3d12526p-1, 0x1.917a6bc29b42cp-4, \
    0x1.0000000000000p+0, 0x0.0p+0, \
    0x1.fd88da3d12526p-1, -0x1.917a6bc29b42cp-4, \
    0x1.f6297cff75cb0p-1, -0x1.8f8b83c69a60bp-3, \
    0x1.e9f4156c62ddap-1, -0x1.294062ed59f06p-2, \
    0x1.d906bcf328d46p-1, -0x1.87de2a6aea963p-2, \
    0x1.c38b2f180bdb1p-1, -0x1.e2b5d3806f63bp-2, \
    0x1.a9b66290ea1a3p-1, -0x1.1c73b39ae68c8p-1, \
    0x1.8bc806b151741p-1, -0x1.44cf325091dd6p-1, \
    0x1.6a09e667f3bcdp-1, -0x1.6a09e667f3bcdp-1, \
    0x1.44cf325091dd6p-1, -0x1.8bc806b151741p-1, \
    0x1.1c73b39ae68c8p-1, -0x1.a9b66290ea1a3p-1, \
    0x1.e2b5d3806f63bp-2, -0x1.c38b2f180bdb1p-1, \
    0x1.87de2a6aea963p-2, -0x1.d906bcf328d46p-1, \
    0x1.294062ed59f06p-2, -0x1.e9f4156c62ddap-1, \
    0x1.8f8b83c69a60bp-3, -0x1.f6297cff75cb0p-1, \
    0x1.917a6bc29b42cp-4, -0x1.fd88da3d12526p-1, \
    0x0.0p+0, -0x1.0000000000000p+0, \
    -0x1.917a6bc29b42cp-4, -0x1.fd88da3d12526p-1, \
    -0x1.8f8b83c69a60bp-3, -0x1.f6297cff75cb0p-1, \
    -0x1.294062ed59f06p-2, -0x1.e9f4156c62ddap-1, \
    -0x1.87de2a6aea963p-2, -0x1.d906bcf328d46p-1, \
    -0x1.e2b5d3806f63bp-2, -0x1.c38b2f180bdb1p-1, \
    -0x1.1c73b39ae68c8p-1, -0x1.a9b66290ea1a3p-1, \
    -0x1.44cf325091dd6p-1, -0x1.8bc806b151741p-1, \
    -0x1.6a09e667f3bcdp-1, -0x1.6a09e667f3bcdp-1, \
    -0x1.8bc806b151741p-1, -0x1.44cf325091dd6p-1, \
    -0x1.a9b66290ea1a3p-1, -0x1.1c73b39ae68c8p-1, \
    -0x1.c38b2f180bdb1p-1, -0x1.e2b5d3806f63bp-2, \
    -0x1.d906bcf328d46p-1, -0x1.87de2a6aea963p-2, \
    -0x1.e9f4156c62ddap-1, -0x1.294062ed59f06p-2, \
    -0x1.f6297cff75cb0p-1, -0x1.8f8b83c69a60bp-3, \
    -0x1.fd88da3d12526p-1, -0x1.917a6bc29b42cp-4, \
    -0x1.0000000000000p+0, 0x0.0p+0, \
    -0x1.fd88da3d12526p-1, 0x1.917a6bc29b42cp-4, \
    -0x1.f6297cff75cb0p-1, 0x1.8f8b83c69a60bp-3, \
    -0x1.e9f4156c62ddap-1, 0x1.294062ed59f06p-2, \
    -0x1.d906bcf328d46p-1, 0x1.87de2a6aea963p-2, \
    -0x1.c38b2f180bdb1p-1, 0x1.e2b5d3806f63bp-2, \
    -0x1.a9b66290ea1a3p-1, 0x1.1c73b39ae68c8p-1, \
    -0x1.8bc806b151741p-1, 0x1.44cf325091dd6p-1, \
    -0x1.6a09e667f3bcdp-1, 0x1.6a09e667f3bcdp-1, \
    -0x1.44cf325091dd6p-1, 0x1.8bc806b151741p-1, \
    -0x1.1c73b39ae68c8p-1, 0x1.a9b66290ea1a3p-1, \
    -0x1.e2b5d3806f63bp-2, 0x1.c38b2f180bdb1p-1, \
    -0x1.87de2a6aea963p-2, 0x1.d906bcf328d46p-1, \
    -0x1.294062ed59f06p-2, 0x1.e9f4156c62ddap-1, \
    -0x1.8f8b83c69a60bp-3, 0x1.f6297cff75cb0p-1, \
    -0x1.917a6bc29b42cp-4, 0x1.fd88da3d12526p-1

#endif
