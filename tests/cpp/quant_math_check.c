/* CPU check of the register quantizer's division-free code paths (neuralnet.cpp_amd/csrc/
 * token_quant.hpp: quantize_code, quantize_exact; the prescale of k_act.hip's k_token_regs)
 * against the exact division they replace (quantize_one: fl(x / s), clamp to +-127, round half
 * away from zero; the reference's per-token absmax quantizer, compute_layer_bitlinear.hpp:443-448).
 *
 * Cases: token scales s = fl(amax * fl(1/127)) over amax from 2^-149 to 2^100, x within 40 ulps
 * of every h * s for half-integers and integers h in [-127.5, 127.5], uniform x in [-amax, amax],
 * and 0, +-amax, NaN, +-inf, subnormal x. Every case must give quantize_one's code: the fast path
 * wherever it does not flag the element, and the exact path always (scales below 2^-100 go
 * through the prescale by 2^100, as the kernel does). Exit status 0 when no case differs. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int q_one(float x, float s)
{
    if (s == 0.0f || isnan(x)) return 0;
    float v = x / s;
    if (isnan(v)) return 0;
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    return (int)roundf(v);
}

static float q_rcp(float s) { return s == 0.0f ? 0.0f : 1.0f / s; }

static int q_code(float x, float r, int* amb)
{
    const float y = x * r;
    const float t = rintf(y);
    *amb |= !(fabsf(y - t) < 0.5f - 0x1p-15f);
    return (int)t;
}

static int q_exact(float x, float s, float r)
{
    const float q0 = x * r;
    const float e = fmaf(-q0, s, x);
    const float v = fmaf(e, r, q0);
    const float a = fminf(fabsf(v), 127.0f);
    float t = rintf(a);
    t = (a - t == 0.5f) ? t + 1.0f : t;
    const int c = (int)t;
    return v != v ? 0 : (signbit(v) ? -c : c);
}

/* the kernel's exact path: prescale x and s by 2^100 below s = 2^-100 */
static int q_exact_token(float x, float s)
{
    const float xs = s < 0x1p-100f ? 0x1p100f : 1.0f;
    const float se = s * xs;
    return q_exact(x * xs, se, q_rcp(se));
}

static uint32_t rng = 12345u;
static uint32_t nxt(void)
{
    rng ^= rng << 13;
    rng ^= rng >> 17;
    rng ^= rng << 5;
    return rng;
}

static long n_cases, n_bad, n_flagged;

static void check(float x, float s, float amax)
{
    if (!(fabsf(x) <= amax) && !isnan(x) && !isinf(x)) return;
    ++n_cases;
    const int ref = q_one(x, s);
    const int ex = q_exact_token(x, s);
    if (ex != ref)
    {
        if (n_bad < 10) printf("exact path: x=%a s=%a code %d, division %d\n", x, s, ex, ref);
        ++n_bad;
    }
    int amb = 0;
    const int c = q_code(x, q_rcp(s), &amb);
    if (amb)
        ++n_flagged;
    else if (c != ref)
    {
        if (n_bad < 10) printf("fast path: x=%a s=%a code %d, division %d\n", x, s, c, ref);
        ++n_bad;
    }
}

int main(int argc, char** argv)
{
    const int n_scales = argc > 1 ? atoi(argv[1]) : 1500;
    for (int si = 0; si < n_scales; ++si)
    {
        const int ex = (int)(nxt() % 250) - 149;
        const float amax = ldexpf(1.0f + (float)(nxt() & 0x7FFFFF) * 0x1p-23f, ex);
        const float s = amax * (1.0f / 127.0f);
        for (int h2 = -255; h2 <= 255; ++h2)
        {
            const float xc = 0.5f * (float)h2 * s;
            for (int k = -40; k <= 40; ++k)
            {
                float x = xc;
                uint32_t b;
                memcpy(&b, &x, 4);
                b += (uint32_t)k;
                memcpy(&x, &b, 4);
                check(x, s, amax);
            }
        }
        for (int k = 0; k < 5000; ++k) check(amax * ((float)(int32_t)nxt() * 0x1p-31f), s, amax);
        const float sp[] = {0.0f, -0.0f, amax, -amax, NAN, 0x1p-149f, -0x1p-149f, 0x1p-140f};
        for (int k = 0; k < 8; ++k) check(sp[k], s, amax);
    }
    /* tokens with an infinite element: amax = inf, s = inf */
    check(1.0f, INFINITY, INFINITY);
    check(INFINITY, INFINITY, INFINITY);
    check(-INFINITY, INFINITY, INFINITY);
    /* all-zero token: s = 0 */
    check(0.0f, 0.0f, 0.0f);
    check(NAN, 0.0f, 0.0f);
    printf("cases %ld, mismatches %ld (fast path flagged %ld)\n", n_cases, n_bad, n_flagged);
    return n_bad ? 1 : 0;
}
