// fpntt.h -- exact NTT butterflies in float64 for moduli near 2^50, and the
// static bound schedule that keeps them exact.
//
// A modulus q <= FP_QMAX (2^50 + 2^29) is handled with words held as
// integer-valued doubles.  Every intermediate is an integer of magnitude
// below 2^53, so every operation below is exact:
//
//   MM(y, w, wq) = y*w - b*q with b = rint(y*wq), wq = fl(w/q), |w| <= q/2
//     h = fl(y*w); l = fma(y, w, -h)     (y*w = h + l exactly)
//     b = rint(fl(y*wq))
//     r = fma(-b, q, h)                  (exact: |r| < 2^53, an integer)
//     t = r + l                          (exact: |t| < 2^53)
//   |b - y*w/q| <= 1/2 + |y|*2^-53*(1+2^-50), hence
//     |t| <= q/2 + |y| * q * 2^-53 * (1+2^-50) <= q/2 + |y|/8 * (1+2^-20)
//   for q <= FP_QMAX, and |r| <= |t| + |l| <= q/2 + |y|*(q/2^53)*1.5 < 2^53.
//
//   RED(x) = fma(-rint(x*qinv), q, x),  qinv = fl(1/q): |RED(x)| <= q/2 + 2
//   for |x| <= 8q.
//
// Bounds are tracked in units of q/1024 (integers, rounded up):
//   MM output  <= 513 + ceil(Y/8)        (Y: bound of |y|)
//   RED output <= 513
//   a value is exact while its bound stays below 2^53 / q * 1024 >= 8191;
//   the schedule below keeps every bound at or below FP_BMAX = 7168 (7q).
//
// Forward (Cooley-Tukey) butterflies X' = X + t, Y' = X - t with t = MM(Y):
// every output has the bound of X plus that of t.  A round whose outputs
// would exceed FP_CT_T reduces its first stage's X inputs instead.
// Inverse (Gentleman-Sande) butterflies X' = X + Y, Y' = MM(X - Y): a sum
// output whose bound would exceed FP_GS_T = FP_BMAX / 2 is reduced (decided
// per register at compile time from the register's history inside the
// round), so that the next sum, formed before any reduction, stays exact.
// Between the two passes of a transform the words are stored as doubles,
// bounded by FP_MID_F (forward: the first pass's last round reduces its X
// inputs if it would exceed it) or FP_GS_T (inverse: every round's outputs
// are unreduced sums <= FP_GS_T or products <= mm(FP_BMAX)).
#pragma once

#define FP_QMAX ((1ull << 50) + (1ull << 29))

namespace fpb {

constexpr long FP_CANON = 1024;  // canonical input [0, q)
constexpr long FP_RED = 513;
constexpr long FP_BMAX = 7168;
constexpr long FP_CT_T = 5120;
constexpr long FP_GS_T = 3584;  // sums of two such values stay <= FP_BMAX
constexpr long FP_MID_F = 4096;

constexpr long mm(long y) { return 513 + (y + 7) / 8; }
constexpr long lmax(long a, long b) { return a > b ? a : b; }

// ---- forward rounds: the bound is the same for every register ----
// bound after nst stages from bin, with or without reducing the first
// stage's X inputs
constexpr long ct_run(int nst, long bin, bool red) {
  long b = bin;
  for (int s = 0; s < nst; s++) b = (s == 0 && red ? FP_RED : b) + mm(b);
  return b;
}
constexpr bool ct_red(int nst, long bin) { return ct_run(nst, bin, false) > FP_CT_T; }
constexpr long ct_out(int nst, long bin) { return ct_run(nst, bin, ct_red(nst, bin)); }
// the largest bound any value reaches inside the round (the round's output)
constexpr bool ct_ok(int nst, long bin) { return ct_out(nst, bin) <= FP_BMAX && bin <= FP_BMAX; }

// ---- inverse rounds: register i of a round of nst stages on W = 2^nst'
// registers (stage s pairs i and i + 2^s for bit s of i clear) ----
// Simulates the round from the uniform input bound bin (<= FP_GS_T).
// Returns, for (s, i) >= 0, whether that sum output is reduced; for s < 0 the
// largest output bound of the round.
constexpr long gs_sim(int nst, int W, long bin, int qs, int qi) {
  if (bin < 0) return -1;
  long b[16] = {};
  for (int i = 0; i < W; i++) b[i] = bin;
  long mx = bin;
  for (int s = 0; s < nst; s++) {
    long nb[16] = {};
    for (int i = 0; i < W; i++) nb[i] = b[i];
    for (int i = 0; i < W; i++) {
      if ((i >> s) & 1) continue;
      const int j = i + (1 << s);
      const long sum = b[i] + b[j];
      const bool red = sum > FP_GS_T;
      if (s == qs && i == qi) return red ? 1 : 0;
      nb[i] = red ? FP_RED : sum;
      nb[j] = mm(sum);
      mx = lmax(mx, lmax(sum, nb[j]));
    }
    for (int i = 0; i < W; i++) b[i] = nb[i];
  }
  if (qs >= 0) return 0;
  long out = 0;
  for (int i = 0; i < W; i++) out = lmax(out, b[i]);
  return (mx > FP_BMAX || bin > FP_GS_T) ? -1 : out;
}
constexpr bool gs_red(int nst, int W, long bin, int s, int i) { return gs_sim(nst, W, bin, s, i) == 1; }
constexpr long gs_out(int nst, int W, long bin) { return gs_sim(nst, W, bin, -1, -1); }

// ---- the rounds of one pass, in execution order ----
// 16-word kernels: forward {4, S-4}, inverse {S-4, 4};
// 8-word kernels: rounds of w8_width(S, k) stages, k = 0.. forward and
// k = .. 0 inverse.
constexpr int w8_nr(int S) { return (S + 2) / 3; }
constexpr int w8_width(int S, int k) { return S - 3 * k < 3 ? S - 3 * k : 3; }
constexpr int round_count(bool w8, int S) { return w8 ? w8_nr(S) : 2; }
constexpr int round_width(bool w8, bool fwd, int S, int r) {
  return w8 ? (fwd ? w8_width(S, r) : w8_width(S, w8_nr(S) - 1 - r)) : (fwd ? (r == 0 ? 4 : S - 4) : (r == 0 ? S - 4 : 4));
}
// Forward pass (first: reads canonical words and stores at most FP_MID_F;
// second: reads at most FP_MID_F): the X-reduction flag (want_red) or the
// input bound of round r; r = round_count gives the pass's output bound.
constexpr long ct_pass(bool w8, int S, bool first, int r, bool want_red) {
  long b = first ? FP_CANON : FP_MID_F;
  const int n = round_count(w8, S);
  for (int k = 0; k < n; k++) {
    const int w = round_width(w8, true, S, k);
    bool red = ct_red(w, b);
    if (first && k == n - 1 && ct_run(w, b, red) > FP_MID_F) red = true;
    if (k == r) return want_red ? (red ? 1 : 0) : b;
    b = ct_run(w, b, red);
  }
  return b;
}
constexpr bool ct_pass_ok(bool w8, int S, bool first) {
  const long out = ct_pass(w8, S, first, round_count(w8, S), false);
  return out <= (first ? FP_MID_F : FP_BMAX);
}
// Inverse pass (first: reads canonical words; second: reads at most
// FP_GS_T): the input bound of round r (-1 if the schedule is not exact);
// r = round_count gives the pass's output bound.
constexpr long gs_pass(bool w8, int S, bool first, int r) {
  long b = first ? FP_CANON : FP_GS_T;
  for (int k = 0; k < r; k++) b = gs_out(round_width(w8, false, S, k), w8 ? 8 : 16, b);
  return b;
}
constexpr bool gs_pass_ok(bool w8, int S, bool first) {
  const long out = gs_pass(w8, S, first, round_count(w8, S));
  return out >= 0 && out <= FP_GS_T;
}

}  // namespace fpb
