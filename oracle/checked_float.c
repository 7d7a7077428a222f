/*
 * TEST INFRASTRUCTURE ONLY — integer-significand checked binary32/binary64 law.
 *
 * CPU restatement of the reference's scalar law; each function names the reference
 * lines it follows (paths relative to the reference's Crates/). It is the checker for the
 * HIP path, never part of it. Values and fault kinds are pinned by the reference's own
 * known-answer tests (tests/golden/scalar_kat.json) and by closed forms in
 * tests/test_oracle_scalar.py (host IEEE RNE for every non-fault value, exact products in
 * double / __float128 for the tiny-after-rounding classification).
 */
#include "oracle.h"

#include <string.h>

typedef unsigned __int128 u128;

/* core/scalar_float_underflow.rs:61-73 */
static int policy_rejects(int policy, int tiny, int inexact, int subnormal)
{
    switch (policy) {
    case ORC_POLICY_IEEE:
        return tiny && inexact;
    case ORC_POLICY_REJECT_SUBNORMAL:
        return subnormal || (tiny && inexact);
    default:
        return 0;
    }
}

/* core/scalar_checked_float.rs:343-351 (identical in f64.rs:129-138) */
static uint64_t jam_right(uint64_t v, uint32_t d)
{
    if (d == 0)
        return v;
    if (d < 64)
        return (v >> d) | (uint64_t)((v & ((1ull << d) - 1)) != 0);
    return (uint64_t)(v != 0);
}

/* f64.rs:140-151 */
static uint64_t jam_right_128(u128 v, uint32_t d)
{
    if (d == 0)
        return (uint64_t)v;
    if (d < 128)
        return (uint64_t)((v >> d) | (u128)((v & (((u128)1 << d) - 1)) != 0));
    return (uint64_t)(v != 0);
}

/* scalar_checked_float.rs:354-356: IEEE 754-2019 4.3.1 ties-to-even */
static int round_up(uint64_t sig, uint64_t discarded)
{
    return discarded > 4 || (discarded == 4 && (sig & 1));
}

/* ====================================================================== binary32 */

typedef struct {
    uint32_t sign;
    int32_t exp;
    uint64_t sig;
} parts;

/* scalar_checked_float.rs:318-340. Returns -1 for a non-finite encoding, 0 for +-0. */
static int decode32(uint32_t bits, parts *p)
{
    uint32_t e = (bits >> 23) & 0xff, f = bits & 0x7fffff;
    if (e == 0xff)
        return -1;
    if (e == 0 && f == 0)
        return 0;
    p->sign = bits >> 31;
    if (e == 0) {
        p->exp = -126;
        p->sig = f;
    } else {
        p->exp = (int32_t)e - 127;
        p->sig = f | 0x800000u;
    }
    return 1;
}

/* scalar_checked_float.rs:376-448. Normalizes ext to [2^26, 2^27), classifies tininess with
 * an unbounded exponent, then packs with the binary32 exponent range. */
static int pack32(uint32_t sign, uint64_t ext, int32_t exp, uint32_t *out, int *tiny,
                  int *inexact, int *subnormal)
{
    while (ext >= (1ull << 27)) {
        ext = jam_right(ext, 1);
        exp += 1;
    }
    while (ext < (1ull << 26)) {
        ext <<= 1;
        exp -= 1;
    }
    {   /* round_to_precision (:361-374) with the exponent unbounded */
        uint64_t s = ext >> 3;
        int32_t ue = exp;
        if (round_up(s, ext & 7))
            s += 1;
        if (s == (1ull << 24))
            ue += 1;
        *tiny = ue < -126;
    }
    if (exp < -126) {
        ext = jam_right(ext, (uint32_t)(-126 - exp));
        exp = -126;
    }
    uint64_t discarded = ext & 7, s = ext >> 3;
    *inexact = discarded != 0;
    if (round_up(s, discarded))
        s += 1;
    if (exp == -126 && s < 0x800000u) {
        *out = (sign << 31) | (uint32_t)s;
        *subnormal = s != 0;
    } else {
        if (s >= (1ull << 24)) {
            s >>= 1;
            exp += 1;
        }
        if (exp > 127)
            return ORC_OVERFLOW;
        *out = (sign << 31) | ((uint32_t)(exp + 127) << 23) | ((uint32_t)s & 0x7fffff);
        *subnormal = 0;
    }
    return ORC_OK;
}

/* scalar_checked_float.rs:508-532 */
static int passthrough32(uint32_t v, int policy, uint32_t *out)
{
    uint32_t mag = v & 0x7fffffffu;
    int sub = mag != 0 && mag < 0x800000u;
    if (policy_rejects(policy, sub, 0, sub))
        return ORC_UNDERFLOW;
    *out = v;
    return ORC_OK;
}

/* scalar_checked_float.rs:450-506 */
static int add32(uint32_t l, uint32_t r, int subtract, int policy, uint32_t *out)
{
    parts a, b;
    int ka = decode32(l, &a);
    if (ka < 0)
        return ORC_INVALID;
    int kb = decode32(r, &b);
    if (kb < 0)
        return ORC_INVALID;
    if (kb > 0)
        b.sign ^= (uint32_t)subtract;
    if (ka == 0) {
        if (kb > 0)
            return passthrough32((b.sign << 31) | (r & 0x7fffffffu), policy, out);
        uint32_t ls = l >> 31, rs = (r >> 31) ^ (uint32_t)subtract;
        *out = (ls == rs) ? (ls << 31) : 0u;
        return ORC_OK;
    }
    if (kb == 0)
        return passthrough32(l, policy, out);
    if (a.exp < b.exp) {
        parts t = a;
        a = b;
        b = t;
    }
    uint64_t ae = a.sig << 3;
    uint64_t be = jam_right(b.sig << 3, (uint32_t)(a.exp - b.exp));
    uint32_t rsign;
    uint64_t ext;
    if (a.sign == b.sign) {
        rsign = a.sign;
        ext = ae + be;
    } else if (ae >= be) {
        rsign = a.sign;
        ext = ae - be;
    } else {
        rsign = b.sign;
        ext = be - ae;
    }
    if (ext == 0) {
        *out = 0;
        return ORC_OK;
    }
    int tiny, inexact, sub;
    uint32_t bits;
    int k = pack32(rsign, ext, a.exp, &bits, &tiny, &inexact, &sub);
    if (k)
        return k;
    if (policy_rejects(policy, tiny, inexact, sub))
        return ORC_UNDERFLOW;
    *out = bits;
    return ORC_OK;
}

/* scalar_checked_float.rs:534-579 */
static int mul32(uint32_t l, uint32_t r, int policy, uint32_t *out)
{
    parts a, b;
    int ka = decode32(l, &a);
    if (ka < 0)
        return ORC_INVALID;
    int kb = decode32(r, &b);
    if (kb < 0)
        return ORC_INVALID;
    if (ka == 0 || kb == 0) {
        *out = ((l ^ r) >> 31) << 31;
        return ORC_OK;
    }
    uint64_t product = a.sig * b.sig;
    int32_t top = 63 - __builtin_clzll(product);
    int32_t exp = a.exp + b.exp + top - 46;
    uint64_t ext = top > 26 ? jam_right(product, (uint32_t)(top - 26)) : product << (26 - top);
    int tiny, inexact, sub;
    uint32_t bits;
    int k = pack32(a.sign ^ b.sign, ext, exp, &bits, &tiny, &inexact, &sub);
    if (k)
        return k;
    if (policy_rejects(policy, tiny, inexact, sub))
        return ORC_UNDERFLOW;
    *out = bits;
    return ORC_OK;
}

/* scalar_checked_float.rs:584-631 */
static int div32(uint32_t l, uint32_t r, int policy, uint32_t *out)
{
    parts a, b;
    int ka = decode32(l, &a);
    if (ka < 0)
        return ORC_INVALID;
    int kb = decode32(r, &b);
    if (kb < 0)
        return ORC_INVALID;
    uint32_t sign = (l ^ r) >> 31;
    if (kb == 0)
        return ORC_DIVIDE_BY_ZERO;
    if (ka == 0) {
        *out = sign << 31;
        return ORC_OK;
    }
    int32_t sa = 23 - (63 - __builtin_clzll(a.sig));
    a.sig <<= sa;
    a.exp -= sa;
    int32_t sb = 23 - (63 - __builtin_clzll(b.sig));
    b.sig <<= sb;
    b.exp -= sb;
    uint64_t num = a.sig;
    int32_t exp = a.exp - b.exp;
    if (num < b.sig) {
        num <<= 1;
        exp -= 1;
    }
    uint64_t scaled = num << 26;
    uint64_t ext = scaled / b.sig;
    if (scaled % b.sig)
        ext |= 1;
    int tiny, inexact, sub;
    uint32_t bits;
    int k = pack32(sign, ext, exp, &bits, &tiny, &inexact, &sub);
    if (k)
        return k;
    if (policy_rejects(policy, tiny, inexact, sub))
        return ORC_UNDERFLOW;
    *out = bits;
    return ORC_OK;
}

/* scalar_checked_float.rs:239-271 */
int orc_neg_f32(uint32_t v, int policy, uint32_t *out)
{
    if ((v & 0x7f800000u) == 0x7f800000u)
        return ORC_INVALID;
    uint32_t res = v ^ 0x80000000u;
    int sub = (res & 0x7fffffffu) != 0 && (res & 0x7f800000u) == 0;
    if (policy_rejects(policy, sub, 0, sub))
        return ORC_UNDERFLOW;
    *out = res;
    return ORC_OK;
}

/* scalar_checked_float.rs:273-309 */
int orc_relu_f32(uint32_t v, int policy, uint32_t *out)
{
    if ((v & 0x7f800000u) == 0x7f800000u)
        return ORC_INVALID;
    uint32_t res = ((v & 0x80000000u) || (v & 0x7fffffffu) == 0) ? 0u : v;
    int sub = res != 0 && (res & 0x7f800000u) == 0;
    if (policy_rejects(policy, sub, 0, sub))
        return ORC_UNDERFLOW;
    *out = res;
    return ORC_OK;
}

/* scalar_checked_float.rs:634-652: both operands finite; strictly positive input selects
 * upstream, else +0; the selected value passes neg(policy) then neg(default policy). */
int orc_relu_backward_f32(uint32_t x, uint32_t up, int policy, uint32_t *out)
{
    if ((x & 0x7f800000u) == 0x7f800000u || (up & 0x7f800000u) == 0x7f800000u)
        return ORC_INVALID;
    int positive = !(x & 0x80000000u) && (x & 0x7fffffffu) != 0;
    uint32_t sel = positive ? up : 0u, t;
    int k = orc_neg_f32(sel, policy, &t);
    if (k)
        return k;
    return orc_neg_f32(t, ORC_POLICY_IEEE, out);
}

int orc_add_f32(uint32_t a, uint32_t b, int policy, uint32_t *out) { return add32(a, b, 0, policy, out); }
int orc_sub_f32(uint32_t a, uint32_t b, int policy, uint32_t *out) { return add32(a, b, 1, policy, out); }
int orc_mul_f32(uint32_t a, uint32_t b, int policy, uint32_t *out) { return mul32(a, b, policy, out); }
int orc_div_f32(uint32_t a, uint32_t b, int policy, uint32_t *out) { return div32(a, b, policy, out); }

/* ====================================================================== binary64 */

#define F64_FRAC_MASK ((1ull << 52) - 1)
#define F64_HIDDEN (1ull << 52)
#define F64_EXT_LO (1ull << 55) /* NORMALIZED_EXTENT (f64.rs:21) */
#define F64_EXT_HI (1ull << 56)

/* f64.rs:103-127 */
static int decode64(uint64_t bits, parts *p)
{
    uint64_t e = (bits >> 52) & 0x7ff, f = bits & F64_FRAC_MASK;
    if (e == 0x7ff)
        return -1;
    if (e == 0 && f == 0)
        return 0;
    p->sign = (uint32_t)(bits >> 63);
    if (e == 0) {
        p->exp = -1022;
        p->sig = f;
    } else {
        p->exp = (int32_t)e - 1023;
        p->sig = f | F64_HIDDEN;
    }
    return 1;
}

/* f64.rs:174-236 */
static int pack64(uint32_t sign, uint64_t ext, int32_t exp, uint64_t *out, int *tiny,
                  int *inexact, int *subnormal)
{
    while (ext >= F64_EXT_HI) {
        ext = jam_right(ext, 1);
        exp += 1;
    }
    while (ext < F64_EXT_LO) {
        ext <<= 1;
        exp -= 1;
    }
    {
        uint64_t s = ext >> 3;
        int32_t ue = exp;
        if (round_up(s, ext & 7))
            s += 1;
        if (s == (1ull << 53))
            ue += 1;
        *tiny = ue < -1022;
    }
    if (exp < -1022) {
        ext = jam_right(ext, (uint32_t)(-1022 - exp));
        exp = -1022;
    }
    uint64_t discarded = ext & 7, s = ext >> 3;
    *inexact = discarded != 0;
    if (round_up(s, discarded))
        s += 1;
    uint64_t sbits = (uint64_t)sign << 63;
    if (exp == -1022 && s < F64_HIDDEN) {
        *out = sbits | s;
        *subnormal = s != 0;
    } else {
        if (s >= (1ull << 53)) {
            s >>= 1;
            exp += 1;
        }
        if (exp > 1023)
            return ORC_OVERFLOW;
        *out = sbits | ((uint64_t)(exp + 1023) << 52) | (s & F64_FRAC_MASK);
        *subnormal = 0;
    }
    return ORC_OK;
}

/* f64.rs:238-262 */
static int passthrough64(uint64_t v, int policy, uint64_t *out)
{
    uint64_t mag = v & ~(1ull << 63);
    int sub = mag != 0 && mag < F64_HIDDEN;
    if (policy_rejects(policy, sub, 0, sub))
        return ORC_UNDERFLOW;
    *out = v;
    return ORC_OK;
}

/* f64.rs:264-324 */
static int add64(uint64_t l, uint64_t r, int subtract, int policy, uint64_t *out)
{
    parts a, b;
    int ka = decode64(l, &a);
    if (ka < 0)
        return ORC_INVALID;
    int kb = decode64(r, &b);
    if (kb < 0)
        return ORC_INVALID;
    if (kb > 0)
        b.sign ^= (uint32_t)subtract;
    if (ka == 0) {
        if (kb > 0)
            return passthrough64(((uint64_t)b.sign << 63) | (r & ~(1ull << 63)), policy, out);
        uint64_t ls = l >> 63, rs = (r >> 63) ^ (uint64_t)subtract;
        *out = (ls == rs) ? (ls << 63) : 0ull;
        return ORC_OK;
    }
    if (kb == 0)
        return passthrough64(l, policy, out);
    if (a.exp < b.exp) {
        parts t = a;
        a = b;
        b = t;
    }
    uint64_t ae = a.sig << 3;
    uint64_t be = jam_right(b.sig << 3, (uint32_t)(a.exp - b.exp));
    uint32_t rsign;
    uint64_t ext;
    if (a.sign == b.sign) {
        rsign = a.sign;
        ext = ae + be;
    } else if (ae >= be) {
        rsign = a.sign;
        ext = ae - be;
    } else {
        rsign = b.sign;
        ext = be - ae;
    }
    if (ext == 0) {
        *out = 0;
        return ORC_OK;
    }
    int tiny, inexact, sub;
    uint64_t bits;
    int k = pack64(rsign, ext, a.exp, &bits, &tiny, &inexact, &sub);
    if (k)
        return k;
    if (policy_rejects(policy, tiny, inexact, sub))
        return ORC_UNDERFLOW;
    *out = bits;
    return ORC_OK;
}

/* f64.rs:326-370 */
static int mul64(uint64_t l, uint64_t r, int policy, uint64_t *out)
{
    parts a, b;
    int ka = decode64(l, &a);
    if (ka < 0)
        return ORC_INVALID;
    int kb = decode64(r, &b);
    if (kb < 0)
        return ORC_INVALID;
    if (ka == 0 || kb == 0) {
        *out = ((l ^ r) >> 63) << 63;
        return ORC_OK;
    }
    u128 product = (u128)a.sig * (u128)b.sig;
    uint64_t hi = (uint64_t)(product >> 64), lo = (uint64_t)product;
    int32_t top = hi ? 127 - __builtin_clzll(hi) : 63 - __builtin_clzll(lo);
    int32_t exp = a.exp + b.exp + top - 104;
    uint64_t ext = top > 55 ? jam_right_128(product, (uint32_t)(top - 55))
                            : (uint64_t)(product << (55 - top));
    int tiny, inexact, sub;
    uint64_t bits;
    int k = pack64(a.sign ^ b.sign, ext, exp, &bits, &tiny, &inexact, &sub);
    if (k)
        return k;
    if (policy_rejects(policy, tiny, inexact, sub))
        return ORC_UNDERFLOW;
    *out = bits;
    return ORC_OK;
}

/* f64.rs:372-431 */
static int div64(uint64_t l, uint64_t r, int policy, uint64_t *out)
{
    parts a, b;
    int ka = decode64(l, &a);
    if (ka < 0)
        return ORC_INVALID;
    int kb = decode64(r, &b);
    if (kb < 0)
        return ORC_INVALID;
    uint32_t sign = (uint32_t)((l ^ r) >> 63);
    if (kb == 0)
        return ORC_DIVIDE_BY_ZERO;
    if (ka == 0) {
        *out = (uint64_t)sign << 63;
        return ORC_OK;
    }
    int32_t sa = 52 - (63 - __builtin_clzll(a.sig));
    a.sig <<= sa;
    a.exp -= sa;
    int32_t sb = 52 - (63 - __builtin_clzll(b.sig));
    b.sig <<= sb;
    b.exp -= sb;
    u128 num = a.sig, den = b.sig;
    int32_t exp = a.exp - b.exp;
    if (num < den) {
        num <<= 1;
        exp -= 1;
    }
    u128 scaled = num << 55;
    uint64_t ext = (uint64_t)(scaled / den);
    if (scaled % den)
        ext |= 1;
    int tiny, inexact, sub;
    uint64_t bits;
    int k = pack64(sign, ext, exp, &bits, &tiny, &inexact, &sub);
    if (k)
        return k;
    if (policy_rejects(policy, tiny, inexact, sub))
        return ORC_UNDERFLOW;
    *out = bits;
    return ORC_OK;
}

/* f64.rs:24-56 */
int orc_neg_f64(uint64_t v, int policy, uint64_t *out)
{
    if ((v & 0x7ff0000000000000ull) == 0x7ff0000000000000ull)
        return ORC_INVALID;
    uint64_t res = v ^ (1ull << 63);
    int sub = (res & ~(1ull << 63)) != 0 && (res & 0x7ff0000000000000ull) == 0;
    if (policy_rejects(policy, sub, 0, sub))
        return ORC_UNDERFLOW;
    *out = res;
    return ORC_OK;
}

/* f64.rs:58-97 */
int orc_relu_f64(uint64_t v, int policy, uint64_t *out)
{
    if ((v & 0x7ff0000000000000ull) == 0x7ff0000000000000ull)
        return ORC_INVALID;
    uint64_t res = ((v >> 63) || (v & ~(1ull << 63)) == 0) ? 0ull : v;
    int sub = res != 0 && (res & 0x7ff0000000000000ull) == 0;
    if (policy_rejects(policy, sub, 0, sub))
        return ORC_UNDERFLOW;
    *out = res;
    return ORC_OK;
}

/* f64.rs:431-448 (PcuCheckedFloat for f64::pcu_checked_relu_backward_with_policy) */
int orc_relu_backward_f64(uint64_t x, uint64_t up, int policy, uint64_t *out)
{
    const uint64_t inf = 0x7ff0000000000000ull;
    if ((x & inf) == inf || (up & inf) == inf)
        return ORC_INVALID;
    int positive = !(x >> 63) && (x & ~(1ull << 63)) != 0;
    uint64_t sel = positive ? up : 0ull, t;
    int k = orc_neg_f64(sel, policy, &t);
    if (k)
        return k;
    return orc_neg_f64(t, ORC_POLICY_IEEE, out);
}

int orc_add_f64(uint64_t a, uint64_t b, int policy, uint64_t *out) { return add64(a, b, 0, policy, out); }
int orc_sub_f64(uint64_t a, uint64_t b, int policy, uint64_t *out) { return add64(a, b, 1, policy, out); }
int orc_mul_f64(uint64_t a, uint64_t b, int policy, uint64_t *out) { return mul64(a, b, policy, out); }
int orc_div_f64(uint64_t a, uint64_t b, int policy, uint64_t *out) { return div64(a, b, policy, out); }

/* ============================================================ exact conversions */

/* core/scalar_checked_conversion/integer/integer.rs:13-46 (pack_count) */
static uint64_t pack_count(uint64_t count, uint32_t fraction_bits, uint32_t bias)
{
    if (count == 0)
        return 0;
    uint32_t exponent = 63 - (uint32_t)__builtin_clzll(count);
    uint64_t sig;
    if (exponent <= fraction_bits) {
        sig = count << (fraction_bits - exponent);
    } else {
        uint32_t shift = exponent - fraction_bits;
        uint64_t q = count >> shift, rem = count & ((1ull << shift) - 1), half = 1ull << (shift - 1);
        sig = q + (uint64_t)(rem > half || (rem == half && (q & 1)));
    }
    if (sig == (1ull << (fraction_bits + 1))) {
        sig >>= 1;
        exponent += 1;
    }
    return ((uint64_t)(exponent + bias) << fraction_bits) | (sig & ((1ull << fraction_bits) - 1));
}

uint32_t orc_u64_to_f32_rne(uint64_t v) { return (uint32_t)pack_count(v, 23, 127); }
uint64_t orc_u64_to_f64_rne(uint64_t v) { return pack_count(v, 52, 1023); }

/* core/scalar_widen.rs:9-37 */
uint64_t orc_f32_to_f64_bits(uint32_t bits)
{
    uint64_t sign = (uint64_t)(bits >> 31) << 63;
    uint32_t e = (bits >> 23) & 0xff, f = bits & 0x7fffff;
    if (e == 0xff)
        return sign | (0x7ffull << 52) | ((uint64_t)f << 29);
    if (e != 0)
        return sign | ((uint64_t)(e + (1023 - 127)) << 52) | ((uint64_t)f << 29);
    if (f == 0)
        return sign;
    uint32_t lead = 31 - (uint32_t)__builtin_clz(f);
    uint64_t sig = (uint64_t)f << (52 - lead);
    return sign | ((uint64_t)(lead + 874) << 52) | (sig & F64_FRAC_MASK);
}

int orc_host_flushes_denormals(void)
{
#if defined(__x86_64__)
    unsigned int csr;
    __asm__ volatile("stmxcsr %0" : "=m"(csr));
    return (csr & 0x8040u) != 0; /* FTZ (bit 15) or DAZ (bit 6) */
#else
    return 0;
#endif
}
