// The node kernel's logarithm (the per-step Nernst potential of an ion whose style
// recomputes it), written out in fewer instructions than the library log, which
// carries extra precision through double-double arithmetic.
//
//   log_pos(x): ln x for a positive normal x.  x = 2^e m with m in [sqrt(1/2), sqrt(2)),
//     s = (m - 1) / (m + 1), ln m = 2 atanh(s) = 2 (s + s^3/3 + s^5/5 + ...); with
//     |s| <= 0.1716 the series to s^23 leaves a remainder below 2^-60 of ln m; ln x =
//     e ln2 + ln m (ln 2 again in two parts).
//
// It is within a few ulps of the correctly rounded result; tests/test_fastmath.py
// measures the error of the host build of this same function (hx_fastmath_log)
// against numpy's log.
#pragma once
#include <cmath>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define HX_HD __host__ __device__
#else
#define HX_HD
#endif

namespace hx {

constexpr double kLn2Hi = 0.69314718055994528623;          // ln 2 rounded to a double
constexpr double kLn2Lo = 2.3190468138462996154e-17;       // ln 2 - kLn2Hi

// ln x for positive, finite, normal x (the caller keeps the other cases out)
HX_HD inline double log_pos(double x) {
    int e;
    double m = frexp(x, &e);                // x = m 2^e, m in [1/2, 1)
    if (m < 0.70710678118654752440) {       // to [sqrt(1/2), sqrt(2))
        m *= 2.0;
        e -= 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double z = s * s;
    double q = 1.0 / 23;
    q = fma(z, q, 1.0 / 21);
    q = fma(z, q, 1.0 / 19);
    q = fma(z, q, 1.0 / 17);
    q = fma(z, q, 1.0 / 15);
    q = fma(z, q, 1.0 / 13);
    q = fma(z, q, 1.0 / 11);
    q = fma(z, q, 1.0 / 9);
    q = fma(z, q, 1.0 / 7);
    q = fma(z, q, 1.0 / 5);
    q = fma(z, q, 1.0 / 3);
    // ln m = 2 s + 2 s z q
    const double lnm = fma(2.0 * s, z * q, 2.0 * s);
    const double de = static_cast<double>(e);
    return fma(de, kLn2Hi, fma(de, kLn2Lo, lnm));
}

}  // namespace hx
