"""Generate the golden fixtures of the exact MFFT matmul from first principles.

Everything here is plain Python integer / Fraction arithmetic, independent of
the oracle and of the reference code:

* products.json -- exact products of small big-integer matrices.  Inputs are
  SplitMix64 limbs in plane-major order (the reference's bigmat_rand,
  src/bigmat.c:21-35); the product is computed on Python ints and written as
  2L+1 base-2^16 limbs, plane-major (src/mfftbench.h:74-82, main.c:171).
  Signed cases read the top limb as int16 (two's complement W-bit entries)
  and write the product mod 2^(16 RL) in two's complement.
* normalize.json -- carry normalisation of int64 coefficient planes
  (src/bigmat.c:48-60): the base-2^16 digits of sum_w acc[w] 2^(16 w) mod
  2^(16 RL).
* fpx.json -- the fp32 embedding (src/fpfixed.c): the exact product of two
  fp32 matrices rounded once to binary32, round-half-even, +0.0 for zero.
* fpx64.json -- the fp64 embedding (src/fpfixed.c:115-173, 292-322).  With V
  the exact product scaled onto the integer grid, the reference keeps the
  window of |V|'s top <= 4 base-2^16 limbs; a window wider than the target
  precision (53 bits for fp64, 63 for long double) is rounded to nearest,
  ties to even, on the exact value (Python's float(Fraction) for fp64), and
  a narrower window is returned as it stands, dropping what lies below it.
  Long double results are written as (sig, ex) with value sig * 2^ex.
* splitmix.json -- the first outputs of SplitMix64 for two seeds.

Run from the repository root:  python tests/golden/gen_golden.py
"""
import json
import math
import os
import struct
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15


def splitmix(seed):
    s = seed
    while True:
        s = (s + GAMMA) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        yield z ^ (z >> 31)


def limbs_rand(n, L, seed):
    g = splitmix(seed)
    return [next(g) & 0xFFFF for _ in range(L * n * n)]


def entry_value(planes, n, L, i, j, signed):
    v = 0
    for u in range(L - 1, -1, -1):
        limb = planes[u * n * n + i * n + j]
        if signed and u == L - 1 and limb & 0x8000:
            limb -= 1 << 16
        v = (v << 16) + limb
    return v


def to_limbs(v, RL):
    m = v % (1 << (16 * RL))
    return [(m >> (16 * w)) & 0xFFFF for w in range(RL)]


def product_case(n, L, seed_a, seed_b, signed):
    A = limbs_rand(n, L, seed_a)
    B = limbs_rand(n, L, seed_b)
    RL = 2 * L + 1
    out = [0] * (RL * n * n)
    Av = [[entry_value(A, n, L, i, k, signed) for k in range(n)] for i in range(n)]
    Bv = [[entry_value(B, n, L, k, j, signed) for j in range(n)] for k in range(n)]
    for i in range(n):
        for j in range(n):
            c = sum(Av[i][k] * Bv[k][j] for k in range(n))
            for w, limb in enumerate(to_limbs(c, RL)):
                out[w * n * n + i * n + j] = limb
    return {"n": n, "L": L, "seed_a": seed_a, "seed_b": seed_b, "signed": signed,
            "RL": RL, "out": out}


def normalize_case(n, nplanes, RL, seed):
    g = splitmix(seed)
    acc = []
    for _ in range(nplanes * n * n):
        r = next(g)
        v = (r >> 3) - (1 << 60)          # signed, |v| < 2^60
        acc.append(v)
    out = [0] * (RL * n * n)
    for e in range(n * n):
        total = sum(acc[w * n * n + e] << (16 * w) for w in range(nplanes))
        for w, limb in enumerate(to_limbs(total, RL)):
            out[w * n * n + e] = limb
    return {"n": n, "nplanes": nplanes, "RL": RL, "acc": acc, "out": out}


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def fp32_rand(count, seed, emin, emax):
    g = splitmix(seed)
    xs = []
    for _ in range(count):
        u = next(g)
        m = 1.0 + ((u >> 40) & 0x7FFFFF) / 8388608.0
        e = emin + u % (emax - emin + 1)
        x = m * 2.0 ** e
        xs.append(-x if u >> 63 else x)
    return [f32(x) for x in xs]


def round_f32(q):
    """Fraction -> nearest binary32 (ties to even); exact zero -> +0.0.
    Normal range only (the fixtures stay inside it)."""
    if q == 0:
        return 0.0
    sign = -1.0 if q < 0 else 1.0
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    while q >= Fraction(2) ** (e + 1):
        e += 1
    while q < Fraction(2) ** e:
        e -= 1
    scaled = q / Fraction(2) ** (e - 23)          # in [2^23, 2^24)
    m = scaled.numerator // scaled.denominator
    rem = scaled - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m & 1):
        m += 1
    if m == 1 << 24:
        m >>= 1
        e += 1
    return sign * float(m) * 2.0 ** (e - 23)


def fpx_case(n, seed_a, seed_b, emin, emax):
    A = fp32_rand(n * n, seed_a, emin, emax)
    B = fp32_rand(n * n, seed_b, emin, emax)
    C = []
    for i in range(n):
        for j in range(n):
            q = sum(Fraction(A[i * n + k]) * Fraction(B[k * n + j]) for k in range(n))
            C.append(round_f32(q))
    bits = [struct.unpack("<I", struct.pack("<f", c))[0] for c in C]
    return {"n": n, "seed_a": seed_a, "seed_b": seed_b, "emin": emin, "emax": emax,
            "A_bits": [struct.unpack("<I", struct.pack("<f", a))[0] for a in A],
            "B_bits": [struct.unpack("<I", struct.pack("<f", b))[0] for b in B],
            "C_bits": bits}


def f64_bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def fp64_rand(count, seed, emin, emax):
    """+-m 2^e with m = 1 + (low 52 bits of u) / 2^52, e = emin + u mod span,
    sign = top bit of u (one splitmix64 draw per value)"""
    g = splitmix(seed)
    xs = []
    for _ in range(count):
        u = next(g)
        m = 1.0 + (u & ((1 << 52) - 1)) / float(1 << 52)
        x = m * 2.0 ** (emin + u % (emax - emin + 1))
        xs.append(-x if u >> 63 else x)
    return xs


def window_decode(q, S, bits):
    """The reference's decode of the exact rational q = C[i][j] on a grid of
    scale 2^S, as (sign, sig, ex) with value sign * sig * 2^ex."""
    V = q * Fraction(2) ** S
    assert V.denominator == 1
    V = V.numerator
    if V == 0:
        return 1, 0, 0, True
    sign = -1 if V < 0 else 1
    V = abs(V)
    blen = V.bit_length()
    h = (blen - 1) // 16                 # top non-zero limb
    k = min(h + 1, 4)
    base = 16 * (h - k + 1)
    tb = blen - base                     # bits in the window
    if tb <= bits:
        return sign, V >> base, base - S, True
    drop = blen - bits
    sig = round(Fraction(V, 1 << drop))  # half-even on the exact value
    if sig >> bits:
        sig >>= 1
        drop += 1
    return sign, sig, drop - S, False


def fpx64_case(A, B, n, force_bits, name):
    C64, sig, ex, trunc = [], [], [], 0
    for i in range(n):
        for j in range(n):
            q = sum(Fraction(A[i * n + k]) * Fraction(B[k * n + j]) for k in range(n))
            # the window's limbs are those of q 2^(SA+SB)
            sg, s53, e53, narrow = window_decode(q, S_of(A, B, n, force_bits), 53)
            v = sg * math.ldexp(float(s53), e53) if s53 else 0.0
            if not narrow and abs(v) >= 2.0 ** -1022:
                assert v == float(q)          # round to nearest, ties to even
            if narrow and Fraction(s53) * Fraction(2) ** e53 != abs(q):
                trunc += 1
            C64.append(f64_bits(v))
            sg, s63, e63, _ = window_decode(q, S_of(A, B, n, force_bits), 63)
            sig.append(sg * s63)
            ex.append(e63)
    return {"name": name, "n": n, "force_bits": force_bits,
            "A_bits": [f64_bits(a) for a in A], "B_bits": [f64_bits(b) for b in B],
            "C64_bits": C64, "ld_sig": sig, "ld_ex": ex, "truncated_f64": trunc}


def S_of(A, B, n, force_bits):
    """SA + SB of the grid (src/fpfixed.c:59-71): force_bits/2 each, or minus
    the smallest exponent of the matrix's entries written as mi 2^e2 with mi
    a 53-bit integer"""
    if force_bits:
        return force_bits
    def lo(X):
        es = [math.frexp(x)[1] - 53 for x in X if x != 0.0]
        return min(es) if es else 0
    return -lo(A) - lo(B)


def fpx64_edges():
    """Hand-made entries, n = 4 (data-sized grid, every entry on it).  B's
    columns pick: row sums, A[i][0] + 3 A[i][1], A[i][2] / 2, nothing.
      C[0][0] = 64 + 2^-47 + 2^-70: a 49-bit window; what lies below it
                (more than half an ulp) is dropped: 64, where rounding to
                nearest would give 64 + 2^-46
      C[1][0] = 1 + 2^-53 (tie, even: 1);  C[1][1] = 1 + 3 2^-53 (tie, odd:
                1 + 2^-51);  C[3][0] = -(1 + 2^-53 + 2^-80) (past the tie:
                -(1 + 2^-52));  C[3][1] = -(1 + 3 2^-53) (-(1 + 2^-51))
      C[2][1] = -4.5 + 4.5: exact zero, +0.0;  C[2][2] = 1.5 2^-1074: the
                subnormal result rounds (ties to even) to 2^-1073"""
    t = 2.0 ** -1074
    A = [64.0, 2.0 ** -47, 2.0 ** -70, 0.0,
         1.0, 2.0 ** -53, 0.0, 0.0,
         -4.5, 1.5, 3 * t, 0.0,
         -1.0, -(2.0 ** -53), 0.0, -(2.0 ** -80)]
    B = [1.0, 1.0, 0.0, 0.0,
         1.0, 3.0, 0.0, 0.0,
         1.0, 0.0, 0.5, 0.0,
         1.0, 0.0, 0.0, 0.0]
    return A, B


def main():
    seed = 12345
    products = []
    for n, L in [(1, 2), (2, 2), (3, 4), (2, 8), (4, 8), (3, 16), (5, 16), (2, 32), (3, 64)]:
        products.append(product_case(n, L, seed, seed ^ 0xABCDEF, False))
    for n, L in [(2, 4), (3, 8), (4, 16), (2, 32)]:
        products.append(product_case(n, L, seed + 1, (seed + 1) ^ 0xABCDEF, True))
    normalize = [normalize_case(3, 5, 8, 99), normalize_case(4, 7, 15, 7)]
    fpx = [fpx_case(3, 11, 22, -20, 20), fpx_case(6, 33, 44, -20, 20), fpx_case(4, 55, 66, -3, 3)]
    fpx64 = [fpx64_case(fp64_rand(9, 71, -20, 20), fp64_rand(9, 72, -20, 20), 3, 0, "rand3"),
             fpx64_case(fp64_rand(16, 73, -30, 30), fp64_rand(16, 74, -30, 30), 4, 2048,
                        "rand4_grid2048"),
             fpx64_case(fp64_rand(25, 75, -300, 300), fp64_rand(25, 76, -300, 300), 5, 0,
                        "rand5_wide"),
             fpx64_case(*fpx64_edges(), 4, 0, "edges")]
    g0, g1 = splitmix(0), splitmix(12345)
    sm = {"seed0": [next(g0) for _ in range(4)], "seed12345": [next(g1) for _ in range(4)]}
    for name, obj in [("products", products), ("normalize", normalize), ("fpx", fpx),
                      ("fpx64", fpx64), ("splitmix", sm)]:
        with open(os.path.join(HERE, f"{name}.json"), "w") as f:
            json.dump(obj, f, separators=(",", ":"))
        print("wrote", name)


if __name__ == "__main__":
    main()
