/* Restatement, in C on the host, of the router kernel's exponential
 * (exp_f32_f64 in candle-moe_amd/csrc/topk_softmax.hip): the same IEEE f64
 * operations in the same order, every multiply-add an explicit fma. The
 * coefficients are passed on the command line (parsed from the kernel source
 * by the test). Every f32 d in [-104, 0] is compared with the CPU oracle's
 * definition, (float)exp((double)d) with glibc's exp; prints the number of
 * inputs and of mismatches. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static double C[15];

static float kernel_exp(float d) {
    const double x = (double)d;
    const double n = rint(x * C[0]);
    double r = fma(-n, C[1], x);
    r = fma(-n, C[2], r);
    double s = C[3];
    for (int i = 4; i < 15; ++i) s = fma(r, s, C[i]);
    const double y = ldexp(fma(s, r, 1.0), (int)n);
    return d < -104.0f ? 0.0f : (float)y;
}

int main(int argc, char** argv) {
    if (argc != 16) {
        fprintf(stderr, "usage: %s c0 .. c14\n", argv[0]);
        return 2;
    }
    for (int i = 0; i < 15; ++i) C[i] = strtod(argv[i + 1], NULL);
    uint32_t lim;
    const float f = -104.0f;
    memcpy(&lim, &f, 4);
    long long n = 0, bad = 0;
#pragma omp parallel for reduction(+ : n, bad) schedule(static, 1 << 16)
    for (long long u = 0x80000000LL; u <= (long long)lim; ++u) {
        const uint32_t b = (uint32_t)u;
        float d;
        memcpy(&d, &b, 4);
        const float a = kernel_exp(d), c = (float)exp((double)d);
        uint32_t ua, uc;
        memcpy(&ua, &a, 4);
        memcpy(&uc, &c, 4);
        ++n;
        bad += ua != uc;
    }
    /* special values: -inf and below the range give +0, NaN stays NaN */
    const float ninf = -INFINITY;
    if (kernel_exp(ninf) != 0.0f || kernel_exp(-1000.0f) != 0.0f || !isnan(kernel_exp(NAN))) ++bad;
    printf("%lld %lld\n", n, bad);
    return 0;
}
