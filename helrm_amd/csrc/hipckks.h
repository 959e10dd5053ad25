// hipckks.h -- internal declarations shared by the HIP kernels and the host
// runtime of the MI355X CKKS backend (not part of the C ABI; see
// include/helrm_hip.h for that).
//
// Data layout in HBM
//   * a polynomial is limb-major u64[rows][N]; every value is canonical in
//     [0, q) of its row's modulus;
//   * ciphertexts and plaintexts are in the NTT domain (bit-reversed
//     evaluation order, psi = g^((q-1)/2N) with g the smallest generator);
//   * a QP polynomial at level l has rows q_0..q_l then p_0..p_{K-1};
//   * linear-transform diagonals and Galois keys are stored pre-multiplied
//     by R = 2^64 mod q ("Montgomery form") so that a lazily accumulated
//     128-bit sum of products needs a single REDC per output word.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint64_t u64;
typedef int64_t i64;
typedef unsigned __int128 u128;

#define HCK_MAXMOD 96
#define HCK_MAXSRC 32

// Per-modulus constants (device table indexed by modulus index:
// 0..L-1 the Q chain, L..L+K-1 the P chain).
struct ModC {
  u64 q;
  u64 qinv;  // -q^-1 mod 2^64
  u64 r2;    // 2^128 mod q
  u64 rmod;  // 2^64 mod q
};

// Row -> modulus mapping for a batch of polynomials:
// rows [0, split) use moduli m0.., rows [split, n) use m1..;
// rows in [skip0, skip1) are left untouched.
struct RowMap {
  int n, split, m0, m1, skip0, skip1;
  __host__ __device__ int nact() const { return n - (skip1 - skip0); }
  __host__ __device__ int row(int r) const { return r < skip0 ? r : r + (skip1 - skip0); }
  __host__ __device__ int mod(int row) const { return row < split ? m0 + row : m1 + (row - split); }
};


#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC__)
__device__ __forceinline__ u64 add_mod(u64 a, u64 b, u64 q) { u64 r = a + b; return r >= q ? r - q : r; }
__device__ __forceinline__ u64 sub_mod(u64 a, u64 b, u64 q) { return a >= b ? a - b : a + q - b; }
__device__ __forceinline__ u64 shoup_mul(u64 x, u64 w, u64 wp, u64 q) {
  u64 qh = __umul64hi(x, wp);
  u64 r = x * w - qh * q;
  return r >= q ? r - q : r;
}
// x >= m ? x - m : x, selecting on the borrow of the 64-bit subtraction
// (four VALU instructions; the compiler's own form adds a 64-bit compare).
__device__ __forceinline__ u64 csub_b(u64 x, u64 m) {
  uint32_t dl, dh;
  u64 b;
  asm("v_sub_co_u32_e64 %[dl], %[b], %[xl], %[ml]\n\t"
      "v_subb_co_u32_e64 %[dh], %[b], %[xh], %[mh], %[b]\n\t"
      "v_cndmask_b32_e64 %[dl], %[dl], %[xl], %[b]\n\t"
      "v_cndmask_b32_e64 %[dh], %[dh], %[xh], %[b]"
      : [dl] "=&v"(dl), [dh] "=&v"(dh), [b] "=&s"(b)
      : [xl] "v"((uint32_t)x), [xh] "v"((uint32_t)(x >> 32)), [ml] "v"((uint32_t)m), [mh] "v"((uint32_t)(m >> 32)));
  return ((u64)dh << 32) | dl;
}
// High 64 bits of y*p in six VALU instructions: the middle column
// yl*ph + yh*pl + hi(yl*pl) is summed with the carry-out of v_mad_u64_u32
// instead of being split into zero-extended halves.
__device__ __forceinline__ u64 mulhi64(u64 y, u64 p) {
  const uint32_t yl = (uint32_t)y, yh = (uint32_t)(y >> 32), pl = (uint32_t)p, ph = (uint32_t)(p >> 32);
  const u64 m1 = (u64)yl * ph + __umulhi(yl, pl);  // < 2^64
  u64 m2, c;
  asm("v_mad_u64_u32 %0, %1, %2, %3, %4" : "=v"(m2), "=s"(c) : "v"(yh), "v"(pl), "v"(m1));
  const u64 r = (u64)yh * ph + (m2 >> 32);  // < 2^64
  uint32_t rh;
  u64 c2;
  asm("v_addc_co_u32_e64 %0, %1, 0, %2, %3" : "=v"(rh), "=s"(c2) : "v"((uint32_t)(r >> 32)), "s"(c));
  return ((u64)rh << 32) | (uint32_t)r;
}
// Shoup product in [0, 2q) for any y < 2^64: y*w + floor(y*wp / 2^64) * nq
// mod 2^64 with nq = 2^64 - q, the low product added through the addend of
// v_mad_u64_u32 (no separate 64-bit subtraction).
__device__ __forceinline__ u64 shoup_lazy(u64 y, u64 w, u64 wp, u64 nq) {
  const u64 Q = mulhi64(y, wp);
  const u64 yw = y * w;
  u64 t, c;
  asm("v_mad_u64_u32 %0, %1, %2, %3, %4" : "=v"(t), "=s"(c) : "v"((uint32_t)Q), "s"((uint32_t)nq), "v"(yw));
  const uint32_t th = (uint32_t)(t >> 32) + (uint32_t)Q * (uint32_t)(nq >> 32) + (uint32_t)(Q >> 32) * (uint32_t)nq;
  return ((u64)th << 32) | (uint32_t)t;
}
// 128-bit lazy accumulator: (hi, lo) += a*b, keeping hi < q (needs q < 2^62).
__device__ __forceinline__ void mac_lazy(u64& lo, u64& hi, u64 a, u64 b, u64 q) {
  u64 plo = a * b, phi = __umul64hi(a, b);
  u64 nlo = lo + plo;
  hi = hi + phi + (nlo < lo ? 1 : 0);
  lo = nlo;
  hi = hi >= q ? hi - q : hi;
}
// Exact sum of up to 16 products of words below 2^62, in column form:
//   sum = s0 + s1*2^32 + (s2 + c0)*2^64 + c1*2^96
// s0 collects a0*b0, s1 collects a0*b1 + a1*b0, s2 collects a1*b1 (32-bit
// halves); c0 and c1 count the carries out of s0 and s1, taken from the
// carry-out of v_mad_u64_u32.  Seven VALU instructions per product (the
// carry reads sit three or more instructions after their writes).  s2 cannot
// overflow: a1, b1 < 2^30, so 16 products stay below 2^64.
struct Acc128 { u64 s0, s1, s2; uint32_t c0, c1; };
__device__ __forceinline__ void acc_zero(Acc128& A) { A.s0 = A.s1 = A.s2 = 0; A.c0 = A.c1 = 0; }
__device__ __forceinline__ void acc_mac(Acc128& A, u64 a, u64 b) {
  const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32), b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
  u64 ca, cb, cc, cd;
  // not volatile: a pure function of its operands, free to be scheduled
  asm(
      "v_mad_u64_u32 %[s0], %[ca], %[a0], %[b0], %[s0]\n\t"
      "v_mad_u64_u32 %[s1], %[cb], %[a0], %[b1], %[s1]\n\t"
      "v_mad_u64_u32 %[s1], %[cc], %[a1], %[b0], %[s1]\n\t"
      "v_mad_u64_u32 %[s2], %[cd], %[a1], %[b1], %[s2]\n\t"
      "v_addc_co_u32_e64 %[c0], %[cd], 0, %[c0], %[ca]\n\t"
      "v_addc_co_u32_e64 %[c1], %[cd], 0, %[c1], %[cb]\n\t"
      "v_addc_co_u32_e64 %[c1], %[cd], 0, %[c1], %[cc]"
      : [s0] "+v"(A.s0), [s1] "+v"(A.s1), [s2] "+v"(A.s2), [c0] "+v"(A.c0), [c1] "+v"(A.c1),
        [ca] "=&s"(ca), [cb] "=&s"(cb), [cc] "=&s"(cc), [cd] "=&s"(cd)
      : [a0] "v"(a0), [a1] "v"(a1), [b0] "v"(b0), [b1] "v"(b1));
}
// The same with b uniform across the wave (held in SGPRs: the constant of a
// basis conversion); each v_mad_u64_u32 reads one SGPR.
__device__ __forceinline__ void acc_mac_s(Acc128& A, u64 a, u64 b) {
  const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32), b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
  u64 ca, cb, cc, cd;
  asm("v_mad_u64_u32 %[s0], %[ca], %[b0], %[a0], %[s0]\n\t"
      "v_mad_u64_u32 %[s1], %[cb], %[b1], %[a0], %[s1]\n\t"
      "v_mad_u64_u32 %[s1], %[cc], %[b0], %[a1], %[s1]\n\t"
      "v_mad_u64_u32 %[s2], %[cd], %[b1], %[a1], %[s2]\n\t"
      "v_addc_co_u32_e64 %[c0], %[cd], 0, %[c0], %[ca]\n\t"
      "v_addc_co_u32_e64 %[c1], %[cd], 0, %[c1], %[cb]\n\t"
      "v_addc_co_u32_e64 %[c1], %[cd], 0, %[c1], %[cc]"
      : [s0] "+v"(A.s0), [s1] "+v"(A.s1), [s2] "+v"(A.s2), [c0] "+v"(A.c0), [c1] "+v"(A.c1),
        [ca] "=&s"(ca), [cb] "=&s"(cb), [cc] "=&s"(cc), [cd] "=&s"(cd)
      : [a0] "v"(a0), [a1] "v"(a1), [b0] "s"(b0), [b1] "s"(b1));
}
// Exact sum of at most 8 products of words below 2^61 (every modulus here is
// below 2^61).  Split at 32 bits the high halves are below 2^29, so a middle
// column of 4 products (8 terms below 2^61) and the top column of 8 products
// (below 2^58 each) cannot overflow: only the low column counts carries, and
// the middle column is kept in two halves (products 0-3 and 4-7).  5 VALU
// instructions per product instead of 7.
struct Acc61 { u64 s0, s1a, s1b, s2; uint32_t c0; };
__device__ __forceinline__ void acc61_zero(Acc61& A) { A.s0 = A.s1a = A.s1b = A.s2 = 0; A.c0 = 0; }
// the first product of an accumulator (and of its second middle half) sets
// the columns instead of adding to zeros
__device__ __forceinline__ void acc61_first_s(Acc61& A, u64 a, u64 b) {
  const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32), b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
  u64 junk;
  asm("v_mad_u64_u32 %[s0], %[j], %[b0], %[a0], 0\n\t"
      "v_mad_u64_u32 %[s1], %[j], %[b1], %[a0], 0\n\t"
      "v_mad_u64_u32 %[s1], %[j], %[b0], %[a1], %[s1]\n\t"
      "v_mad_u64_u32 %[s2], %[j], %[b1], %[a1], 0"
      : [s0] "=&v"(A.s0), [s1] "=&v"(A.s1a), [s2] "=&v"(A.s2), [j] "=&s"(junk)
      : [a0] "v"(a0), [a1] "v"(a1), [b0] "s"(b0), [b1] "s"(b1));
  A.c0 = 0;
}
__device__ __forceinline__ void acc61_first_half_s(Acc61& A, u64 a, u64 b) {
  const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32), b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
  u64 ca, junk;
  asm("v_mad_u64_u32 %[s0], %[ca], %[b0], %[a0], %[s0]\n\t"
      "v_mad_u64_u32 %[s1], %[j], %[b1], %[a0], 0\n\t"
      "v_mad_u64_u32 %[s1], %[j], %[b0], %[a1], %[s1]\n\t"
      "v_mad_u64_u32 %[s2], %[j], %[b1], %[a1], %[s2]\n\t"
      "v_addc_co_u32_e64 %[c0], %[j], 0, %[c0], %[ca]"
      : [s0] "+v"(A.s0), [s1] "=&v"(A.s1b), [s2] "+v"(A.s2), [c0] "+v"(A.c0), [ca] "=&s"(ca), [j] "=&s"(junk)
      : [a0] "v"(a0), [a1] "v"(a1), [b0] "s"(b0), [b1] "s"(b1));
}
template <int HALF>
__device__ __forceinline__ void acc61_mac_s(Acc61& A, u64 a, u64 b) {
  const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32), b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
  u64& s1 = HALF ? A.s1b : A.s1a;
  u64 ca, junk;
  asm("v_mad_u64_u32 %[s0], %[ca], %[b0], %[a0], %[s0]\n\t"
      "v_mad_u64_u32 %[s1], %[j], %[b1], %[a0], %[s1]\n\t"
      "v_mad_u64_u32 %[s1], %[j], %[b0], %[a1], %[s1]\n\t"
      "v_mad_u64_u32 %[s2], %[j], %[b1], %[a1], %[s2]\n\t"
      "v_addc_co_u32_e64 %[c0], %[j], 0, %[c0], %[ca]"
      : [s0] "+v"(A.s0), [s1] "+v"(s1), [s2] "+v"(A.s2), [c0] "+v"(A.c0), [ca] "=&s"(ca), [j] "=&s"(junk)
      : [a0] "v"(a0), [a1] "v"(a1), [b0] "s"(b0), [b1] "s"(b1));
}
__device__ __forceinline__ void acc61_value(const Acc61& A, u64& lo, u64& hi) {
  const u64 s1 = A.s1a + A.s1b;
  const u64 s1c = s1 < A.s1a ? 1 : 0;
  const u64 t = s1 << 32;
  lo = A.s0 + t;
  hi = A.s2 + A.c0 + (s1 >> 32) + (s1c << 32) + (lo < t ? 1 : 0);
}
// REDC(value of A) - sub mod q for an Acc61 whose value is below q * 2^64
// (8 products of words below 2^61 and a column bound kept by the caller), sub
// < q: the columns are combined, reduced and corrected in 32-bit carry
// chains (about 33 VALU instructions where the 64-bit form takes ~47):
//   s1 = s1a + s1b (carry s1c); lo = s0 + s1 * 2^32 (carry c1);
//   hi = s2 + s1 / 2^32 + s1c * 2^32 + c0 + c1;
//   m = lo * qinv mod 2^64 (qinv = -q^-1); t = hi + mulhi(m, q) + (lo != 0);
//   r = t >= q ? t - q : t;  result = r - sub (+ q if it borrows).
__device__ __forceinline__ u64 acc61_redc_sub(const Acc61& A, u64 q, u64 qinv, u64 sub) {
  uint32_t lol, loh, hil, hih;
  {
    uint32_t s1l, s1h;
    u64 k0, k1, k2, k3, s1c, c1;
    asm("v_add_co_u32_e64 %[s1l], %[k0], %[al], %[bl]\n\t"
        "v_addc_co_u32_e64 %[s1h], %[s1c], %[ah], %[bh], %[k0]\n\t"
        "v_add_co_u32_e64 %[loh], %[c1], %[s0h], %[s1l]\n\t"
        "v_add_co_u32_e64 %[hil], %[k1], %[s2l], %[s1h]\n\t"
        "v_addc_co_u32_e64 %[hih], %[k1], %[s2h], 0, %[k1]\n\t"
        "v_addc_co_u32_e64 %[hih], %[k1], %[hih], 0, %[s1c]\n\t"
        "v_add_co_u32_e64 %[hil], %[k2], %[hil], %[c0]\n\t"
        "v_addc_co_u32_e64 %[hih], %[k2], %[hih], 0, %[k2]\n\t"
        "v_addc_co_u32_e64 %[hil], %[k3], %[hil], 0, %[c1]\n\t"
        "v_addc_co_u32_e64 %[hih], %[k3], %[hih], 0, %[k3]"
        : [s1l] "=&v"(s1l), [s1h] "=&v"(s1h), [loh] "=&v"(loh), [hil] "=&v"(hil), [hih] "=&v"(hih),
          [k0] "=&s"(k0), [k1] "=&s"(k1), [k2] "=&s"(k2), [k3] "=&s"(k3), [s1c] "=&s"(s1c), [c1] "=&s"(c1)
        : [al] "v"((uint32_t)A.s1a), [ah] "v"((uint32_t)(A.s1a >> 32)), [bl] "v"((uint32_t)A.s1b),
          [bh] "v"((uint32_t)(A.s1b >> 32)), [s0h] "v"((uint32_t)(A.s0 >> 32)), [s2l] "v"((uint32_t)A.s2),
          [s2h] "v"((uint32_t)(A.s2 >> 32)), [c0] "v"(A.c0));
    lol = (uint32_t)A.s0;
  }
  const u64 lo = ((u64)loh << 32) | lol;
  // m = lo * qinv mod 2^64
  const uint32_t ql = (uint32_t)q, qh = (uint32_t)(q >> 32), il = (uint32_t)qinv, ih = (uint32_t)(qinv >> 32);
  const u64 p0 = (u64)lol * il;
  const uint32_t mh = (uint32_t)(p0 >> 32) + lol * ih + loh * il;
  const u64 m = ((u64)mh << 32) | (uint32_t)p0;
  const u64 mq = mulhi64(m, q);
  uint32_t tl, th, rl, rh, dl, dh;
  u64 cz, k4, b0, b1;
  // t = hi + mq + (lo != 0); r = t - q unless that borrows; d = r - sub, + q if that borrows
  asm("v_cmp_ne_u64_e64 %[cz], 0, %[lo]\n\t"
      "v_addc_co_u32_e64 %[tl], %[k4], %[hil], %[mql], %[cz]\n\t"
      "v_addc_co_u32_e64 %[th], %[k4], %[hih], %[mqh], %[k4]\n\t"
      "v_sub_co_u32_e64 %[rl], %[b0], %[tl], %[ql]\n\t"
      "v_subb_co_u32_e64 %[rh], %[b0], %[th], %[qh], %[b0]\n\t"
      "v_cndmask_b32_e64 %[rl], %[rl], %[tl], %[b0]\n\t"
      "v_cndmask_b32_e64 %[rh], %[rh], %[th], %[b0]\n\t"
      "v_sub_co_u32_e64 %[dl], %[b1], %[rl], %[sl]\n\t"
      "v_subb_co_u32_e64 %[dh], %[b1], %[rh], %[sh], %[b1]\n\t"
      "v_cndmask_b32_e64 %[tl], 0, %[ql], %[b1]\n\t"
      "v_cndmask_b32_e64 %[th], 0, %[qh], %[b1]\n\t"
      "v_add_co_u32_e64 %[dl], %[k4], %[dl], %[tl]\n\t"
      "v_addc_co_u32_e64 %[dh], %[k4], %[dh], %[th], %[k4]"
      : [tl] "=&v"(tl), [th] "=&v"(th), [rl] "=&v"(rl), [rh] "=&v"(rh), [dl] "=&v"(dl), [dh] "=&v"(dh),
        [cz] "=&s"(cz), [k4] "=&s"(k4), [b0] "=&s"(b0), [b1] "=&s"(b1)
      : [lo] "v"(lo), [hil] "v"(hil), [hih] "v"(hih), [mql] "v"((uint32_t)mq), [mqh] "v"((uint32_t)(mq >> 32)),
        [ql] "v"(ql), [qh] "v"(qh), [sl] "v"((uint32_t)sub), [sh] "v"((uint32_t)(sub >> 32)));
  return ((u64)dh << 32) | dl;
}
// One destination word of a basis extension from at most 8 sources:
// REDC(sum_i y(i) * h[i]) - sub mod q, y(i) < 2^61 (zero past the job's
// sources) and h[i] < q the row's table words (Montgomery form, read for all
// 8 i: the table holds spare words past its last row).
template <class Y>
__device__ __forceinline__ u64 bconv_word8(Y y, const u64* __restrict__ h, u64 q, u64 qinv, u64 sub) {
  Acc61 A;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    if (i == 0) acc61_first_s(A, y(i), h[i]);
    else if (i < 4) acc61_mac_s<0>(A, y(i), h[i]);
    else if (i == 4) acc61_first_half_s(A, y(i), h[i]);
    else acc61_mac_s<1>(A, y(i), h[i]);
  }
  return acc61_redc_sub(A, q, qinv, sub);
}
// the 128-bit value (lo, hi) of an accumulator
__device__ __forceinline__ void acc_value(const Acc128& A, u64& lo, u64& hi) {
  const u64 t = A.s1 << 32;
  lo = A.s0 + t;
  hi = A.s2 + A.c0 + (A.s1 >> 32) + ((u64)A.c1 << 32) + (lo < t ? 1 : 0);
}
// Montgomery reduction of T = hi*2^64 + lo < q*2^64: returns T * 2^-64 mod q.
__device__ __forceinline__ u64 redc(u64 lo, u64 hi, u64 q, u64 qinv) {
  u64 m = lo * qinv;
  u64 t = hi + mulhi64(m, q) + (lo != 0 ? 1 : 0);
  return csub_b(t, q);
}
__device__ __forceinline__ u64 mont_mul(u64 a, u64 bR, u64 q, u64 qinv) {
  return redc(a * bR, __umul64hi(a, bR), q, qinv);
}
#endif
