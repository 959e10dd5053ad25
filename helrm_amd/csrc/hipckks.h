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

struct RowList {
  int n;
  short row[HCK_MAXMOD];
  short mod[HCK_MAXMOD];
};

#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC__)
__device__ __forceinline__ u64 add_mod(u64 a, u64 b, u64 q) { u64 r = a + b; return r >= q ? r - q : r; }
__device__ __forceinline__ u64 sub_mod(u64 a, u64 b, u64 q) { return a >= b ? a - b : a + q - b; }
__device__ __forceinline__ u64 shoup_mul(u64 x, u64 w, u64 wp, u64 q) {
  u64 qh = __umul64hi(x, wp);
  u64 r = x * w - qh * q;
  return r >= q ? r - q : r;
}
// 128-bit lazy accumulator: (hi, lo) += a*b, keeping hi < q (needs q < 2^62).
__device__ __forceinline__ void mac_lazy(u64& lo, u64& hi, u64 a, u64 b, u64 q) {
  u64 plo = a * b, phi = __umul64hi(a, b);
  u64 nlo = lo + plo;
  hi = hi + phi + (nlo < lo ? 1 : 0);
  lo = nlo;
  hi = hi >= q ? hi - q : hi;
}
// Montgomery reduction of T = hi*2^64 + lo < q*2^64: returns T * 2^-64 mod q.
__device__ __forceinline__ u64 redc(u64 lo, u64 hi, u64 q, u64 qinv) {
  u64 m = lo * qinv;
  u64 t = hi + __umul64hi(m, q) + (lo != 0 ? 1 : 0);
  return t >= q ? t - q : t;
}
__device__ __forceinline__ u64 mont_mul(u64 a, u64 bR, u64 q, u64 qinv) {
  return redc(a * bR, __umul64hi(a, bR), q, qinv);
}
#endif
