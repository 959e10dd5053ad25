// ntt.hip -- negacyclic NTT / inverse NTT for gfx950.
//
// Transform of one limb of N = 2^logN words, N = R x C with R = 2^SA rows of
// C = 2^SB columns (5 <= SA, SB <= 8).  Forward (Cooley-Tukey, distances
// N/2 .. 1, twiddle W[(N + g) >> (lt + 1)] for the pair (g, g + 2^lt)):
//   pass A  distances N/2 .. C      (column sub-transforms of size R)
//   pass B  distances C/2 .. 1      (row sub-transforms of size C)
// Inverse (Gentleman-Sande, distances 1 .. N/2, then N^-1): pass B, pass A.
//
// A sub-transform of size 2^S is computed by 2^(S-4) threads holding 16
// words each in registers: one radix-16 round (4 butterfly stages without
// any exchange), one LDS exchange, one round of the remaining S-4 stages.
// Launches over few limbs use kernels with 8 words per thread instead
// (rounds of 3 stages, twice the waves per limb).
// Butterflies are lazy (Harvey): forward values stay in [0, 4q), inverse
// values in [0, 2q); each pass's output is reduced to [0, q) only where the
// transform ends, so the result equals the textbook NTT word for word.
// Twiddles are (w, floor(w 2^64 / q)) pairs read as one 16-byte load.
//
// Limbs whose modulus is at most FP_QMAX (the 40- and 50-bit primes) run the
// same passes on float64 words instead: exact products by the float64
// multiply-add (fpntt.h), so a butterfly costs 8 VALU instructions on the
// full-rate FP64 pipe instead of ~19 integer ones.  Twiddles of such a
// modulus are (w, fl(w / q)) float64 pairs, w centred; words between the two
// passes are integer-valued doubles, and each transform still reads and
// writes canonical u64 residues.
#include <algorithm>

#include "fpntt.h"
#include "hipckks.h"
#include "kernels.h"

namespace {

constexpr int NTT_TPB = 256;

__device__ __forceinline__ u64 csub(u64 x, u64 m) { return csub_b(x, m); }

// Twiddle slots of a round of NST stages over 16 registers: 8 + 4 + ...
__host__ __device__ constexpr int ntt_round_slots(int nst) { return nst == 0 ? 0 : (16 >> nst) + ntt_round_slots(nst - 1); }

// The twiddles of one register round, loaded ahead of its butterflies so the
// loads are in flight together (slot order: stages in execution order,
// twiddles k = 0 .. within a stage).
template <int NST>
struct RoundTw { uint4 t[ntt_round_slots(NST)]; };

// Element i of the round stands for global index g_i = A + B + (i << ls) with
// B < 2^ls and A a multiple of 2^(ls+4): the pair at register distance rd
// uses twiddle ((N + A) >> (ls + log2(rd) + 1)) + (i >> (log2(rd) + 1)).
template <bool FWD, int NST>
__device__ __forceinline__ void round_tw_load(RoundTw<NST>& T, u64 A, int ls, u64 Nn, const uint4* __restrict__ tw) {
  int sl = 0;
#pragma unroll
  for (int s = 0; s < NST; s++) {
    const int lrd = FWD ? NST - 1 - s : s;
    const int sh = lrd + 1;
    const u64 tb = (Nn + A) >> (ls + sh);
#pragma unroll
    for (int k = 0; k < (16 >> sh); k++, sl++) T.t[sl] = tw[tb + k];
  }
}
// A round over 16 consecutive words of a row, from the lane-interleaved
// table: tab points at entry [r][0][j] of a [R][slots][P] table, slot sl of
// lane j is tab[sl * P], so each load of a wave is one contiguous read.
template <int NST>
__device__ __forceinline__ void round_tw_load_tab(RoundTw<NST>& T, const uint4* __restrict__ tab, int P) {
#pragma unroll
  for (int sl = 0; sl < ntt_round_slots(NST); sl++) T.t[sl] = tab[(size_t)sl * P];
}
// NST butterfly stages on v[W]; tw_at(s, k, sl) gives twiddle k of stage s
// (slot sl of the round): a preloaded RoundTw in the 16-word kernels, a load
// per stage in the 8-word ones.
template <bool FWD, int NST, int W = 16, class TWF>
__device__ __forceinline__ void ntt_round_f(u64 (&v)[W], TWF tw_at, u64 q) {
  const u64 q2 = q + q, q4 = q2 + q2, nq = 0 - q;
  int sl = 0;
#pragma unroll
  for (int s = 0; s < NST; s++) {
    const int lrd = FWD ? NST - 1 - s : s;  // log2 of the register distance
    const int rd = 1 << lrd;
    const int sh = lrd + 1;
    uint4 ts[W >> 1];
#pragma unroll
    for (int k = 0; k < (W >> sh); k++) ts[k] = tw_at(s, k, sl + k);
#pragma unroll
    for (int k = 0; k < (W >> sh); k++, sl++) {
      const uint4 t4 = ts[k];
      const u64 w = ((u64)t4.y << 32) | t4.x, wp = ((u64)t4.w << 32) | t4.z;
#pragma unroll
      for (int r = 0; r < rd; r++) {
        const int i = (k << sh) + r;
        u64 X = v[i], Y = v[i + rd];
        if (FWD) {
          // Harvey butterflies with the reduction of X on every other stage
          // (q < 2^61): a reducing stage takes X < 8q to x < 4q and leaves
          // outputs < 6q, the next one skips it and leaves outputs < 8q; the
          // last stage of every round reduces, so rounds start below 6q.
          const bool reduce = ((NST - 1 - s) & 1) == 0;
          const u64 x = reduce ? csub(X, q4) : X;
          const u64 t = shoup_lazy(Y, w, wp, nq);
          v[i] = x + t;
          v[i + rd] = x + q2 - t;
        } else {
          v[i] = csub(X + Y, q2);
          v[i + rd] = shoup_lazy(X + q2 - Y, w, wp, nq);
        }
      }
    }
  }
}
// NST butterfly stages on v[16] with the preloaded twiddles.
template <bool FWD, int NST>
__device__ __forceinline__ void ntt_round(u64 (&v)[16], const RoundTw<NST>& T, u64 q) {
  ntt_round_f<FWD, NST>(v, [&](int, int, int sl) { return T.t[sl]; }, q);
}

// ---- float64 words (moduli q <= FP_QMAX; fpntt.h gives the bounds) ----
__device__ __forceinline__ double f_val(u64 bits) { return __longlong_as_double((long long)bits); }
__device__ __forceinline__ u64 f_bits(double x) { return (u64)__double_as_longlong(x); }
// a canonical residue (< 2^52) as a double: its bits under the exponent of
// 2^52, minus 2^52
__device__ __forceinline__ double f_in(u64 x) { return f_val(x | 0x4330000000000000ull) - 4503599627370496.0; }
// y * w - rint(y * wq) * q, exact (|t| <= q/2 + |y|/8)
__device__ __forceinline__ double f_mm(double y, double w, double wq, double q) {
  const double h = y * w;
  const double l = __fma_rn(y, w, -h);
  const double b = __builtin_rint(y * wq);
  const double r = __fma_rn(-b, q, h);
  return r + l;
}
// x - rint(x / q) * q, in [-q/2 - 2, q/2 + 2]
__device__ __forceinline__ double f_red(double x, double q, double qinv) {
  return __fma_rn(-__builtin_rint(x * qinv), q, x);
}
// the canonical residue of x as a u64: 2^52 + (x mod q) is below 2^53, so
// its bits under the exponent of 2^52 are the residue
__device__ __forceinline__ u64 f_canon(double x, const FpC& c) {
  const double r = f_red(x, c.q, c.qinv);
  const double s = r + (r < 0.0 ? c.cneg : 4503599627370496.0);
  return f_bits(s) - 0x4330000000000000ull;
}
__device__ __forceinline__ double2 f_tw(const uint4& t) {
  return make_double2(f_val(((u64)t.y << 32) | t.x), f_val(((u64)t.w << 32) | t.z));
}
// NST forward (Cooley-Tukey) stages on W registers: X' = X + t, Y' = X - t,
// t = MM(Y); RED reduces the first stage's X inputs.
template <int NST, int W, bool RED, class TWF>
__device__ __forceinline__ void f_round_fwd(double (&v)[W], TWF tw_at, const FpC& c) {
  int sl = 0;
#pragma unroll
  for (int s = 0; s < NST; s++) {
    const int lrd = NST - 1 - s;
    const int rd = 1 << lrd;
    const int sh = lrd + 1;
    double2 ts[W >> 1];
#pragma unroll
    for (int k = 0; k < (W >> sh); k++) ts[k] = f_tw(tw_at(s, k, sl + k));
#pragma unroll
    for (int k = 0; k < (W >> sh); k++, sl++) {
#pragma unroll
      for (int r = 0; r < rd; r++) {
        const int i = (k << sh) + r;
        double X = v[i];
        if (RED && s == 0) X = f_red(X, c.q, c.qinv);
        const double t = f_mm(v[i + rd], ts[k].x, ts[k].y, c.q);
        v[i] = X + t;
        v[i + rd] = X - t;
      }
    }
  }
}
// Which sum outputs of an inverse round are reduced (fpb::gs_red), as a
// table the unrolled loops index with constants.
template <int NST, int W, long BIN>
struct GsPlan {
  bool red[4][16];
  constexpr GsPlan() : red() {
    for (int s = 0; s < NST; s++)
      for (int i = 0; i < W; i++) red[s][i] = fpb::gs_red(NST, W, BIN, s, i);
  }
};
// NST inverse (Gentleman-Sande) stages on W registers from the input bound
// BIN: X' = X + Y (reduced where the plan says), Y' = MM(X - Y); NINV makes
// the round's last stage X' = MM(X + Y, N^-1), Y' = MM(X - Y, w N^-1).
template <int NST, int W, long BIN, bool NINV, class TWF>
__device__ __forceinline__ void f_round_inv(double (&v)[W], TWF tw_at, const FpC& c) {
  static_assert(fpb::gs_out(NST, W, BIN) >= 0, "float64 inverse round out of bounds");
  constexpr GsPlan<NST, W, BIN> plan{};
  int sl = 0;
#pragma unroll
  for (int s = 0; s < NST; s++) {
    const int rd = 1 << s;
    const int sh = s + 1;
    const bool last = NINV && s == NST - 1;
    double2 ts[W >> 1];
    if (!last) {
#pragma unroll
      for (int k = 0; k < (W >> sh); k++) ts[k] = f_tw(tw_at(s, k, sl + k));
    }
#pragma unroll
    for (int k = 0; k < (W >> sh); k++, sl++) {
#pragma unroll
      for (int r = 0; r < rd; r++) {
        const int i = (k << sh) + r;
        const double X = v[i], Y = v[i + rd];
        if (last) {
          v[i] = f_mm(X + Y, c.ni, c.niq, c.q);
          v[i + rd] = f_mm(X - Y, c.wn, c.wnq, c.q);
        } else {
          const double d = X - Y;
          double sum = X + Y;
          if (plan.red[s][i]) sum = f_red(sum, c.q, c.qinv);
          v[i] = sum;
          v[i + rd] = f_mm(d, ts[k].x, ts[k].y, c.q);
        }
      }
    }
  }
}

// LDS column swizzle for the row pass: conflict-free both for the strided
// (j + P*i) and the consecutive (16*j + i) access patterns.
__device__ __forceinline__ int swz(int col) { return col ^ ((col >> 4) & 15); }

// One limb of a batched transform: word offset from the data base and
// modulus index.  Either listed explicitly (rows of several digits of a
// decomposition in one launch) or derived from (RowMap, batch stride).
struct LimbRef { int64_t off; int mod; int pad; };  // pad: batch entry (RowMap path)

// ModDown epilogue of a forward transform (the transform of the extension of
// [x]_P to Q): instead of the transform v, the row pass writes
//   out[b][row][d] = (x[b][row][pos] - v) * P^-1 (+ add[b][row][pos]) (+ acc[b][row][d]),
// d = perm^-1(pos), so the extension never goes back to memory.
struct ModDownEpi {
  const u64* x; size_t x_bstride;       // Q rows of the QP polynomial
  u64* out; size_t o_bstride;
  const u64* add; size_t a_bstride; int add_batches;
  const uint32_t* perm_inv;             // nullptr: identity
  const u64 *pinv, *pinvp;              // [mod] P^-1 mod q and its Shoup companion
  const u64* acc; size_t c_bstride;     // nullptr, or added at the output position (out != acc)
  // scaled pair (launch_ntt_rescale_pair): batch entry b = 2 g + p reads part
  // p of x, multiplies it by ks's K_g of its row, adds C_g to part 0 and
  // writes group g to out (g = 0) or out2 (g = 1); ks == nullptr: off
  const u64* ks; int ks_rows; u64* out2;
};

struct NttArgs {
  const LimbRef* list;  // nullptr: limb y = (row y / batch of rm, batch entry y % batch)
  const u64* src;  // input of the first pass (src == data: in place)
  size_t sstride;
  u64* data;       // output; the second pass works in place on it
  size_t bstride;
  RowMap rm;
  const uint4* tw;   // [mod][N] (w, w') pairs, forward or inverse table
  const uint4* twr;  // [mod][R][slots][P] lane-interleaved twiddles of the row pass's consecutive round
  const ModC* mods;
  const u64 *ninv, *ninvp;  // [mod]
  const FpC* fpc;           // [mod] float64 constants (moduli q <= FP_QMAX)
  int logN, SA, SB, nsub;   // nsub: sub-transforms per workgroup
  int rows;                 // rm.nact()
  int batch;
  int epi;                  // forward row pass ends with the ModDown epilogue
  ModDownEpi e;
};

// Limbs of one modulus are consecutive (row-major over the batch) so that
// the workgroups in flight share few twiddle tables and those stay in L2.
__device__ __forceinline__ LimbRef limb_ref(const NttArgs& a, int y) {
  if (a.list) return a.list[y];
  const int ri = y / a.batch, b = y - ri * a.batch, r = a.rm.row(ri);
  LimbRef l;
  l.off = (int64_t)b * (int64_t)a.bstride + ((int64_t)r << a.logN);
  l.mod = a.rm.mod(r);
  l.pad = b;
  return l;
}
// src offset of the same limb (first pass of an out-of-place transform)
__device__ __forceinline__ int64_t limb_src_off(const NttArgs& a, int y, const LimbRef& l) {
  if (a.list) return l.off;
  return (int64_t)l.pad * (int64_t)a.sstride + (l.off - (int64_t)l.pad * (int64_t)a.bstride);
}

// Column pass (pass A): workgroup = nsub columns x R rows.
template <bool FWD, int S>
__device__ __forceinline__ void ntt_col_int(const NttArgs& a, u64* sm, const LimbRef& lr) {
  // forward: first pass (reads a.src); inverse: second pass (in place)
  constexpr int P = 1 << (S - 4);
  const int nsub = a.nsub;
  const int tid = threadIdx.x;
  const int c = tid & (nsub - 1);
  const int j = tid / nsub;  // in [0, P)
  const int m = lr.mod;
  const u64 q = a.mods[m].q;
  const u64 Nn = 1ull << a.logN;
  const int SB = a.SB;
  const size_t C = (size_t)1 << SB;
  const int col = blockIdx.x * nsub + c;
  u64* poly = a.data + lr.off + col;
  const uint4* tw = a.tw + (size_t)m * Nn;
  u64 v[16];
  if (FWD) {
    const u64* in = a.src + limb_src_off(a, blockIdx.y, lr) + col;
    // round 1: rows j + P*i, distances R/2 .. R/16 rows
    RoundTw<4> T1;
    round_tw_load<true, 4>(T1, 0, S - 4 + SB, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = in[(size_t)(j + P * i) * C];
    ntt_round<true, 4>(v, T1, q);
    RoundTw<S - 4> T2;
    round_tw_load<true, S - 4>(T2, (u64)(16 * j) << SB, SB, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) sm[(j + P * i) * nsub + c] = v[i];
    __syncthreads();
    // round 2: rows 16*j + i, the remaining S-4 stages
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = sm[(16 * j + i) * nsub + c];
    ntt_round<true, S - 4>(v, T2, q);
#pragma unroll
    for (int i = 0; i < 16; i++) poly[(size_t)(16 * j + i) * C] = v[i];
  } else {
    // round 1: rows 16*j + i, distances C .. 2^(S-5) C
    RoundTw<S - 4> T1;
    round_tw_load<false, S - 4>(T1, (u64)(16 * j) << SB, SB, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = poly[(size_t)(16 * j + i) * C];
    ntt_round<false, S - 4>(v, T1, q);
    RoundTw<4> T2;
    round_tw_load<false, 4>(T2, 0, S - 4 + SB, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) sm[(16 * j + i) * nsub + c] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = sm[(j + P * i) * nsub + c];
    ntt_round<false, 4>(v, T2, q);
    const u64 ni = a.ninv[m], nip = a.ninvp[m];
#pragma unroll
    for (int i = 0; i < 16; i++) poly[(size_t)(j + P * i) * C] = csub(shoup_lazy(v[i], ni, nip, 0 - q), q);
  }
}
// The same pass with float64 words (q <= FP_QMAX): canonical words in,
// doubles bounded by the mid-transform bound out (forward), or doubles in and
// canonical words out with N^-1 folded into the last stage (inverse).
template <bool FWD, int S>
__device__ __forceinline__ void ntt_col_fp(const NttArgs& a, u64* sm, const LimbRef& lr) {
  constexpr int P = 1 << (S - 4);
  const int nsub = a.nsub;
  const int tid = threadIdx.x;
  const int c = tid & (nsub - 1);
  const int j = tid / nsub;
  const int m = lr.mod;
  const FpC fc = a.fpc[m];
  const u64 Nn = 1ull << a.logN;
  const int SB = a.SB;
  const size_t C = (size_t)1 << SB;
  const int col = blockIdx.x * nsub + c;
  u64* poly = a.data + lr.off + col;
  const uint4* tw = a.tw + (size_t)m * Nn;
  double v[16];
  if (FWD) {
    static_assert(fpb::ct_pass_ok(false, S, true), "float64 forward column pass out of bounds");
    constexpr bool R1 = fpb::ct_pass(false, S, true, 0, true), R2 = fpb::ct_pass(false, S, true, 1, true);
    const u64* in = a.src + limb_src_off(a, blockIdx.y, lr) + col;
    RoundTw<4> T1;
    round_tw_load<true, 4>(T1, 0, S - 4 + SB, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = f_in(in[(size_t)(j + P * i) * C]);
    f_round_fwd<4, 16, R1>(v, [&](int, int, int sl) { return T1.t[sl]; }, fc);
    RoundTw<S - 4> T2;
    round_tw_load<true, S - 4>(T2, (u64)(16 * j) << SB, SB, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) sm[(j + P * i) * nsub + c] = f_bits(v[i]);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = f_val(sm[(16 * j + i) * nsub + c]);
    f_round_fwd<S - 4, 16, R2>(v, [&](int, int, int sl) { return T2.t[sl]; }, fc);
#pragma unroll
    for (int i = 0; i < 16; i++) poly[(size_t)(16 * j + i) * C] = f_bits(v[i]);
  } else {
    static_assert(fpb::gs_pass_ok(false, S, false), "float64 inverse column pass out of bounds");
    constexpr long B0 = fpb::gs_pass(false, S, false, 0), B1 = fpb::gs_pass(false, S, false, 1);
    RoundTw<S - 4> T1;
    round_tw_load<false, S - 4>(T1, (u64)(16 * j) << SB, SB, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = f_val(poly[(size_t)(16 * j + i) * C]);
    f_round_inv<S - 4, 16, B0, false>(v, [&](int, int, int sl) { return T1.t[sl]; }, fc);
    RoundTw<4> T2;
    round_tw_load<false, 4>(T2, 0, S - 4 + SB, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) sm[(16 * j + i) * nsub + c] = f_bits(v[i]);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = f_val(sm[(j + P * i) * nsub + c]);
    f_round_inv<4, 16, B1, true>(v, [&](int, int, int sl) { return T2.t[sl]; }, fc);
#pragma unroll
    for (int i = 0; i < 16; i++) poly[(size_t)(j + P * i) * C] = f_canon(v[i], fc);
  }
}
template <bool FWD, int S>
__global__ __launch_bounds__(NTT_TPB) void ntt_col_kernel(NttArgs a) {
  __shared__ u64 sm[4096];
  const LimbRef lr = limb_ref(a, blockIdx.y);
  // one modulus per workgroup: the branch is uniform
  if (a.mods[lr.mod].q <= FP_QMAX) ntt_col_fp<FWD, S>(a, sm, lr);
  else ntt_col_int<FWD, S>(a, sm, lr);
}

// Last part of the forward row pass: the canonical transform of one row is in
// srow (consecutive positions, swizzled); store it, or apply the ModDown
// epilogue to it.
template <int S, bool EPI>
__device__ __forceinline__ void row_fwd_tail(const NttArgs& a, const u64* srow, const LimbRef& lr, int r, int j, u64* poly) {
  constexpr int P = 1 << (S - 4);
  constexpr int C = 1 << S;
  const int m = lr.mod;
  const u64 q = a.mods[m].q;
  if (EPI) {
    // ModDown epilogue: limb (batch b, Q row) of the extension
    const int b = lr.pad, row = (int)((lr.off - (int64_t)b * (int64_t)a.bstride) >> a.logN);
    const size_t rowoff = ((size_t)row << a.logN) + (size_t)r * C;
    const int g = a.e.ks ? b >> 1 : 0, part = a.e.ks ? b & 1 : b;
    const u64* xr = a.e.x + (size_t)part * a.e.x_bstride + rowoff;
    const u64* ar = (a.e.add && b < a.e.add_batches) ? a.e.add + (size_t)b * a.e.a_bstride + rowoff : nullptr;
    u64* orow = (g ? a.e.out2 : a.e.out) + (size_t)part * a.e.o_bstride + ((size_t)row << a.logN);
    const u64 pi = a.e.pinv[m], pip = a.e.pinvp[m];
    // every load of the epilogue is issued before the first use, so the
    // latencies overlap instead of adding up word by word
    u64 xv[16], av[16];
    uint32_t dst[16];
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = __builtin_nontemporal_load(&xr[j + P * i]);
    if (ar) {
#pragma unroll
      for (int i = 0; i < 16; i++) av[i] = __builtin_nontemporal_load(&ar[j + P * i]);
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) av[i] = 0;
    }
    if (a.e.perm_inv) {
#pragma unroll
      for (int i = 0; i < 16; i++) dst[i] = a.e.perm_inv[r * C + j + P * i];
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) dst[i] = (uint32_t)(r * C + j + P * i);
    }
    if (a.e.acc) {
      // a sum of the result and acc: acc at the output position, gathered
      // through the same permutation as the stores
      const u64* crow = a.e.acc + (size_t)b * a.e.c_bstride + ((size_t)row << a.logN);
#pragma unroll
      for (int i = 0; i < 16; i++) av[i] = add_mod(av[i], crow[dst[i]], q);
    }
    if (a.e.ks) {
      const int R = a.e.ks_rows;
      const u64 kw = a.e.ks[(size_t)g * R + row], kwp = a.e.ks[(size_t)(2 + g) * R + row];
      const u64 cadd = part == 0 ? a.e.ks[(size_t)(4 + g) * R + row] : 0;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        xv[i] = shoup_mul(xv[i], kw, kwp, q);
        av[i] = add_mod(av[i], cadd, q);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int pos = j + P * i;
      const u64 o = shoup_mul(sub_mod(xv[i], srow[swz(pos)], q), pi, pip, q);
      __builtin_nontemporal_store(add_mod(o, av[i], q), &orow[dst[i]]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) __builtin_nontemporal_store(srow[swz(j + P * i)], &poly[j + P * i]);
  }
}

// Row pass (pass B): workgroup = nsub rows x C columns.
template <bool FWD, int S, bool EPI>
__device__ __forceinline__ void ntt_row_int(const NttArgs& a, u64* sm, const LimbRef& lr) {
  constexpr int P = 1 << (S - 4);
  constexpr int C = 1 << S;
  const int tid = threadIdx.x;
  const int j = tid & (P - 1);
  const int rho = tid >> (S - 4);
  const int m = lr.mod;
  const u64 q = a.mods[m].q;
  const u64 Nn = 1ull << a.logN;
  const int r = blockIdx.x * a.nsub + rho;  // row of the R x C view
  u64* poly = a.data + lr.off + (size_t)r * C;
  u64* srow = sm + rho * C;
  const uint4* tw = a.tw + (size_t)m * Nn;
  constexpr int NSL = ntt_round_slots(S - 4);
  const uint4* twr = a.twr + (((size_t)m * (Nn >> S) + r) * NSL) * P + j;
  const u64 A = (u64)r * C;
  u64 v[16];
  if (FWD) {
    RoundTw<4> T1;
    round_tw_load<true, 4>(T1, A, S - 4, Nn, tw);
    // data words are touched once per pass: streamed past L2 so the twiddle
    // table, shared by every limb of a modulus in the launch, stays cached
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = __builtin_nontemporal_load(&poly[j + P * i]);
    ntt_round<true, 4>(v, T1, q);
#pragma unroll
    for (int i = 0; i < 16; i++) srow[swz(j + P * i)] = v[i];
    __syncthreads();
    // second round's twiddles issued after the barrier (fewer live registers)
    RoundTw<S - 4> T2;
    round_tw_load_tab<S - 4>(T2, twr, P);
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = srow[swz(16 * j + i)];
    ntt_round<true, S - 4>(v, T2, q);
    const u64 q2 = q + q;
#pragma unroll
    for (int i = 0; i < 16; i++) srow[swz(16 * j + i)] = csub(csub(csub(v[i], q2 + q2), q2), q);
    __syncthreads();
    row_fwd_tail<S, EPI>(a, srow, lr, r, j, poly);
  } else {
    const u64* in = a.src + limb_src_off(a, blockIdx.y, lr) + (size_t)r * C;
    // all 16 loads in flight before the LDS writes; the first round's
    // twiddles are issued behind them and arrive during the barrier
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = __builtin_nontemporal_load(&in[j + P * i]);
#pragma unroll
    for (int i = 0; i < 16; i++) srow[swz(j + P * i)] = v[i];
    RoundTw<S - 4> T1;
    round_tw_load_tab<S - 4>(T1, twr, P);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = srow[swz(16 * j + i)];
    ntt_round<false, S - 4>(v, T1, q);
    RoundTw<4> T2;
    round_tw_load<false, 4>(T2, A, S - 4, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) srow[swz(16 * j + i)] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = srow[swz(j + P * i)];
    ntt_round<false, 4>(v, T2, q);
#pragma unroll
    for (int i = 0; i < 16; i++) __builtin_nontemporal_store(v[i], &poly[j + P * i]);
  }
}
template <bool FWD, int S, bool EPI>
__device__ __forceinline__ void ntt_row_fp(const NttArgs& a, u64* sm, const LimbRef& lr) {
  constexpr int P = 1 << (S - 4);
  constexpr int C = 1 << S;
  const int tid = threadIdx.x;
  const int j = tid & (P - 1);
  const int rho = tid >> (S - 4);
  const int m = lr.mod;
  const FpC fc = a.fpc[m];
  const u64 Nn = 1ull << a.logN;
  const int r = blockIdx.x * a.nsub + rho;
  u64* poly = a.data + lr.off + (size_t)r * C;
  u64* srow = sm + rho * C;
  const uint4* tw = a.tw + (size_t)m * Nn;
  constexpr int NSL = ntt_round_slots(S - 4);
  const uint4* twr = a.twr + (((size_t)m * (Nn >> S) + r) * NSL) * P + j;
  const u64 A = (u64)r * C;
  double v[16];
  if (FWD) {
    static_assert(fpb::ct_pass_ok(false, S, false), "float64 forward row pass out of bounds");
    constexpr bool R1 = fpb::ct_pass(false, S, false, 0, true), R2 = fpb::ct_pass(false, S, false, 1, true);
    RoundTw<4> T1;
    round_tw_load<true, 4>(T1, A, S - 4, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = f_val(__builtin_nontemporal_load(&poly[j + P * i]));
    f_round_fwd<4, 16, R1>(v, [&](int, int, int sl) { return T1.t[sl]; }, fc);
#pragma unroll
    for (int i = 0; i < 16; i++) srow[swz(j + P * i)] = f_bits(v[i]);
    __syncthreads();
    RoundTw<S - 4> T2;
    round_tw_load_tab<S - 4>(T2, twr, P);
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = f_val(srow[swz(16 * j + i)]);
    f_round_fwd<S - 4, 16, R2>(v, [&](int, int, int sl) { return T2.t[sl]; }, fc);
#pragma unroll
    for (int i = 0; i < 16; i++) srow[swz(16 * j + i)] = f_canon(v[i], fc);
    __syncthreads();
    row_fwd_tail<S, EPI>(a, srow, lr, r, j, poly);
  } else {
    static_assert(fpb::gs_pass_ok(false, S, true), "float64 inverse row pass out of bounds");
    constexpr long B0 = fpb::gs_pass(false, S, true, 0), B1 = fpb::gs_pass(false, S, true, 1);
    const u64* in = a.src + limb_src_off(a, blockIdx.y, lr) + (size_t)r * C;
    u64 w[16];
#pragma unroll
    for (int i = 0; i < 16; i++) w[i] = __builtin_nontemporal_load(&in[j + P * i]);
#pragma unroll
    for (int i = 0; i < 16; i++) srow[swz(j + P * i)] = w[i];
    RoundTw<S - 4> T1;
    round_tw_load_tab<S - 4>(T1, twr, P);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = f_in(srow[swz(16 * j + i)]);
    f_round_inv<S - 4, 16, B0, false>(v, [&](int, int, int sl) { return T1.t[sl]; }, fc);
    RoundTw<4> T2;
    round_tw_load<false, 4>(T2, A, S - 4, Nn, tw);
#pragma unroll
    for (int i = 0; i < 16; i++) srow[swz(16 * j + i)] = f_bits(v[i]);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = f_val(srow[swz(j + P * i)]);
    f_round_inv<4, 16, B1, false>(v, [&](int, int, int sl) { return T2.t[sl]; }, fc);
#pragma unroll
    for (int i = 0; i < 16; i++) __builtin_nontemporal_store(f_bits(v[i]), &poly[j + P * i]);
  }
}
template <bool FWD, int S, bool EPI = false>
__global__ __launch_bounds__(NTT_TPB) void ntt_row_kernel(NttArgs a) {
  __shared__ u64 sm[4096];
  const LimbRef lr = limb_ref(a, blockIdx.y);
  if (a.mods[lr.mod].q <= FP_QMAX) ntt_row_fp<FWD, S, EPI>(a, sm, lr);
  else ntt_row_int<FWD, S, EPI>(a, sm, lr);
}

// ---------------------------------------------------------------------------
// 8 words per thread, for launches of few limbs.  A sub-transform of 2^S
// points is computed by T = 2^(S-3) threads in rounds of at most 3 stages
// (ceil(S/3) rounds, an LDS exchange between rounds): twice the waves of the
// 16-word kernels per limb and half the instruction chain per wave, so a
// launch over a few dozen limbs keeps more SIMDs busy.  Forward round k acts
// on element bits [ls_k, ls_k + width_k) with ls_k = max(0, S - 3(k+1)),
// width_k = min(3, S - 3k); register i of thread t holds element
//   e = ((t >> ls_k) << (ls_k + 3)) | (i << ls_k) | (t & (2^ls_k - 1)).
// The inverse runs the same rounds in the opposite order.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int w8_ls(int S, int k) { return S - 3 * (k + 1) > 0 ? S - 3 * (k + 1) : 0; }
__host__ __device__ constexpr int w8_width(int S, int k) { return S - 3 * k < 3 ? S - 3 * k : 3; }
__device__ __forceinline__ int w8_elem(int ls, int t, int i) {
  return ((t >> ls) << (ls + 3)) | (i << ls) | (t & ((1 << ls) - 1));
}
// LDS position of element e inside a row (bijection on [0, 2^S), S >= 4):
// XOR of bits 3..6 into bits 0..3 keeps all three access patterns of the
// 256-point row pass free of bank conflicts.
__device__ __forceinline__ int w8_swz(int e) { return e ^ ((e >> 3) & 15); }

// One round k of the 8-word transform: element e of the sub-transform stands
// for global index base + e * stride (stride = 2^lstride); twiddle pairs as
// in round_tw_load with A the element-block base of the thread.
template <bool FWD, int S, int K>
__device__ __forceinline__ void w8_round(u64 (&v)[8], int t, u64 base, int lstride, u64 Nn, const uint4* __restrict__ tw,
                                         u64 q) {
  constexpr int ls = w8_ls(S, K), width = w8_width(S, K);
  if constexpr (width > 0) {
    const u64 A = base + ((u64)((t >> ls) << (ls + 3)) << lstride);
    const int LS = ls + lstride;
    ntt_round_f<FWD, width, 8>(v, [&](int st, int k, int) {
      const int sh = (FWD ? width - 1 - st : st) + 1;
      return tw[((Nn + A) >> (LS + sh)) + k];
    }, q);
  }
}
// The same round on float64 words.  Forward: FIRST selects the pass (the
// first reads canonical words); inverse: NINV folds N^-1 into the round's
// last stage (the transform's last).  The round's place in its pass (r, in
// execution order) fixes its bound schedule.
template <bool FWD, int S, int K, bool FIRST, bool NINV = false>
__device__ __forceinline__ void w8_round_fp(double (&v)[8], int t, u64 base, int lstride, u64 Nn,
                                            const uint4* __restrict__ tw, const FpC& fc) {
  constexpr int ls = w8_ls(S, K), width = w8_width(S, K);
  constexpr int r = FWD ? K : fpb::w8_nr(S) - 1 - K;
  if constexpr (width > 0) {
    const u64 A = base + ((u64)((t >> ls) << (ls + 3)) << lstride);
    const int LS = ls + lstride;
    auto tw_at = [&](int st, int k, int) {
      const int sh = (FWD ? width - 1 - st : st) + 1;
      return tw[((Nn + A) >> (LS + sh)) + k];
    };
    if constexpr (FWD) {
      f_round_fwd<width, 8, fpb::ct_pass(true, S, FIRST, r, true) != 0>(v, tw_at, fc);
    } else {
      f_round_inv<width, 8, fpb::gs_pass(true, S, FIRST, r), NINV>(v, tw_at, fc);
    }
  }
}

// Column pass, 8 words per thread: workgroup = nsub columns x R rows, T
// threads per column (512 threads for 16 columns).
template <bool FWD, int S>
__device__ __forceinline__ void ntt_col8_int(const NttArgs& a, u64* sm, const LimbRef& lr) {
  constexpr int NR = (S + 2) / 3;
  const int nsub = a.nsub;
  const int tid = threadIdx.x;
  const int c = tid & (nsub - 1);
  const int t = tid / nsub;  // in [0, T)
  const int m = lr.mod;
  const u64 q = a.mods[m].q;
  const u64 Nn = 1ull << a.logN;
  const int SB = a.SB;
  const size_t C = (size_t)1 << SB;
  const int col = blockIdx.x * nsub + c;
  u64* poly = a.data + lr.off + col;
  const uint4* tw = a.tw + (size_t)m * Nn;
  u64 v[8];
  if (FWD) {
    const u64* in = a.src + limb_src_off(a, blockIdx.y, lr) + col;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = in[(size_t)w8_elem(w8_ls(S, 0), t, i) * C];
    w8_round<true, S, 0>(v, t, 0, SB, Nn, tw, q);
#pragma unroll
    for (int k = 1; k < NR; k++) {
      const int lp = w8_ls(S, k - 1), lc = w8_ls(S, k);
      if (k > 1) __syncthreads();  // the previous exchange has been read
#pragma unroll
      for (int i = 0; i < 8; i++) sm[w8_elem(lp, t, i) * nsub + c] = v[i];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = sm[w8_elem(lc, t, i) * nsub + c];
      if (k == 1) w8_round<true, S, 1>(v, t, 0, SB, Nn, tw, q);
      if (k == 2) w8_round<true, S, 2>(v, t, 0, SB, Nn, tw, q);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) poly[(size_t)w8_elem(w8_ls(S, NR - 1), t, i) * C] = v[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = poly[(size_t)w8_elem(w8_ls(S, NR - 1), t, i) * C];
#pragma unroll
    for (int k = NR - 1; k >= 0; k--) {
      if (k < NR - 1) {
        const int lp = w8_ls(S, k + 1), lc = w8_ls(S, k);
        if (k < NR - 2) __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) sm[w8_elem(lp, t, i) * nsub + c] = v[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = sm[w8_elem(lc, t, i) * nsub + c];
      }
      if (k == 2) w8_round<false, S, 2>(v, t, 0, SB, Nn, tw, q);
      if (k == 1) w8_round<false, S, 1>(v, t, 0, SB, Nn, tw, q);
      if (k == 0) w8_round<false, S, 0>(v, t, 0, SB, Nn, tw, q);
    }
    const u64 ni = a.ninv[m], nip = a.ninvp[m];
#pragma unroll
    for (int i = 0; i < 8; i++) poly[(size_t)w8_elem(w8_ls(S, 0), t, i) * C] = csub(shoup_lazy(v[i], ni, nip, 0 - q), q);
  }
}
template <bool FWD, int S>
__device__ __forceinline__ void ntt_col8_fp(const NttArgs& a, u64* sm, const LimbRef& lr) {
  constexpr int NR = (S + 2) / 3;
  static_assert(FWD ? fpb::ct_pass_ok(true, S, true) : fpb::gs_pass_ok(true, S, false),
                "float64 8-word column pass out of bounds");
  const int nsub = a.nsub;
  const int tid = threadIdx.x;
  const int c = tid & (nsub - 1);
  const int t = tid / nsub;
  const int m = lr.mod;
  const FpC fc = a.fpc[m];
  const u64 Nn = 1ull << a.logN;
  const int SB = a.SB;
  const size_t C = (size_t)1 << SB;
  const int col = blockIdx.x * nsub + c;
  u64* poly = a.data + lr.off + col;
  const uint4* tw = a.tw + (size_t)m * Nn;
  double v[8];
  if (FWD) {
    const u64* in = a.src + limb_src_off(a, blockIdx.y, lr) + col;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = f_in(in[(size_t)w8_elem(w8_ls(S, 0), t, i) * C]);
    w8_round_fp<true, S, 0, true>(v, t, 0, SB, Nn, tw, fc);
#pragma unroll
    for (int k = 1; k < NR; k++) {
      const int lp = w8_ls(S, k - 1), lc = w8_ls(S, k);
      if (k > 1) __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) sm[w8_elem(lp, t, i) * nsub + c] = f_bits(v[i]);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = f_val(sm[w8_elem(lc, t, i) * nsub + c]);
      if (k == 1) w8_round_fp<true, S, 1, true>(v, t, 0, SB, Nn, tw, fc);
      if (k == 2) w8_round_fp<true, S, 2, true>(v, t, 0, SB, Nn, tw, fc);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) poly[(size_t)w8_elem(w8_ls(S, NR - 1), t, i) * C] = f_bits(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = f_val(poly[(size_t)w8_elem(w8_ls(S, NR - 1), t, i) * C]);
#pragma unroll
    for (int k = NR - 1; k >= 0; k--) {
      if (k < NR - 1) {
        const int lp = w8_ls(S, k + 1), lc = w8_ls(S, k);
        if (k < NR - 2) __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) sm[w8_elem(lp, t, i) * nsub + c] = f_bits(v[i]);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = f_val(sm[w8_elem(lc, t, i) * nsub + c]);
      }
      if (k == 2) w8_round_fp<false, S, 2, false>(v, t, 0, SB, Nn, tw, fc);
      if (k == 1) w8_round_fp<false, S, 1, false>(v, t, 0, SB, Nn, tw, fc);
      if (k == 0) w8_round_fp<false, S, 0, false, true>(v, t, 0, SB, Nn, tw, fc);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) poly[(size_t)w8_elem(w8_ls(S, 0), t, i) * C] = f_canon(v[i], fc);
  }
}
template <bool FWD, int S>
__global__ __launch_bounds__(512) void ntt_col8_kernel(NttArgs a) {
  __shared__ u64 sm[4096];
  const LimbRef lr = limb_ref(a, blockIdx.y);
  if (a.mods[lr.mod].q <= FP_QMAX) ntt_col8_fp<FWD, S>(a, sm, lr);
  else ntt_col8_int<FWD, S>(a, sm, lr);
}

// Last part of the 8-word forward row pass: the canonical row is in srow
// (swizzled by w8_swz); store it, or apply the ModDown epilogue to it.
template <int S, bool EPI>
__device__ __forceinline__ void row8_fwd_tail(const NttArgs& a, const u64* srow, const LimbRef& lr, int r, int t, u64* poly) {
  constexpr int C = 1 << S;
  constexpr int L0 = w8_ls(S, 0);
  const int m = lr.mod;
  const u64 q = a.mods[m].q;
  if (EPI) {
    const int b = lr.pad, row = (int)((lr.off - (int64_t)b * (int64_t)a.bstride) >> a.logN);
    const size_t rowoff = ((size_t)row << a.logN) + (size_t)r * C;
    const int g = a.e.ks ? b >> 1 : 0, part = a.e.ks ? b & 1 : b;
    const u64* xr = a.e.x + (size_t)part * a.e.x_bstride + rowoff;
    const u64* ar = (a.e.add && b < a.e.add_batches) ? a.e.add + (size_t)b * a.e.a_bstride + rowoff : nullptr;
    u64* orow = (g ? a.e.out2 : a.e.out) + (size_t)part * a.e.o_bstride + ((size_t)row << a.logN);
    const u64 pi = a.e.pinv[m], pip = a.e.pinvp[m];
    u64 xv[8], av[8];
    uint32_t dst[8];
#pragma unroll
    for (int i = 0; i < 8; i++) xv[i] = __builtin_nontemporal_load(&xr[w8_elem(L0, t, i)]);
    if (ar) {
#pragma unroll
      for (int i = 0; i < 8; i++) av[i] = __builtin_nontemporal_load(&ar[w8_elem(L0, t, i)]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) av[i] = 0;
    }
    if (a.e.perm_inv) {
#pragma unroll
      for (int i = 0; i < 8; i++) dst[i] = a.e.perm_inv[r * C + w8_elem(L0, t, i)];
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) dst[i] = (uint32_t)(r * C + w8_elem(L0, t, i));
    }
    if (a.e.acc) {
      const u64* crow = a.e.acc + (size_t)b * a.e.c_bstride + ((size_t)row << a.logN);
#pragma unroll
      for (int i = 0; i < 8; i++) av[i] = add_mod(av[i], crow[dst[i]], q);
    }
    if (a.e.ks) {
      const int R = a.e.ks_rows;
      const u64 kw = a.e.ks[(size_t)g * R + row], kwp = a.e.ks[(size_t)(2 + g) * R + row];
      const u64 cadd = part == 0 ? a.e.ks[(size_t)(4 + g) * R + row] : 0;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        xv[i] = shoup_mul(xv[i], kw, kwp, q);
        av[i] = add_mod(av[i], cadd, q);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int pos = w8_elem(L0, t, i);
      const u64 o = shoup_mul(sub_mod(xv[i], srow[w8_swz(pos)], q), pi, pip, q);
      __builtin_nontemporal_store(add_mod(o, av[i], q), &orow[dst[i]]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int pos = w8_elem(L0, t, i);
      __builtin_nontemporal_store(srow[w8_swz(pos)], &poly[pos]);
    }
  }
}

// Row pass, 8 words per thread: workgroup = nsub rows x C columns, T threads
// per row.  Global memory is read and written in the round-0 element order
// (consecutive lanes, consecutive words); the other rounds go through LDS.
template <bool FWD, int S, bool EPI>
__device__ __forceinline__ void ntt_row8_int(const NttArgs& a, u64* sm, const LimbRef& lr) {
  constexpr int T = 1 << (S - 3), C = 1 << S, NR = (S + 2) / 3;
  constexpr int L0 = w8_ls(S, 0), LL = w8_ls(S, NR - 1);
  const int tid = threadIdx.x;
  const int t = tid & (T - 1);
  const int rho = tid >> (S - 3);
  const int m = lr.mod;
  const u64 q = a.mods[m].q;
  const u64 Nn = 1ull << a.logN;
  const int r = blockIdx.x * a.nsub + rho;  // row of the R x C view
  u64* poly = a.data + lr.off + (size_t)r * C;
  u64* srow = sm + rho * C;
  const uint4* tw = a.tw + (size_t)m * Nn;
  const u64 A = (u64)r * C;
  u64 v[8];
  if (FWD) {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = __builtin_nontemporal_load(&poly[w8_elem(L0, t, i)]);
    w8_round<true, S, 0>(v, t, A, 0, Nn, tw, q);
#pragma unroll
    for (int k = 1; k < NR; k++) {
      const int lp = w8_ls(S, k - 1), lc = w8_ls(S, k);
      if (k > 1) __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) srow[w8_swz(w8_elem(lp, t, i))] = v[i];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = srow[w8_swz(w8_elem(lc, t, i))];
      if (k == 1) w8_round<true, S, 1>(v, t, A, 0, Nn, tw, q);
      if (k == 2) w8_round<true, S, 2>(v, t, A, 0, Nn, tw, q);
    }
    // canonical values back in round-0 order for coalesced stores
    const u64 q2 = q + q;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) srow[w8_swz(w8_elem(LL, t, i))] = csub(csub(csub(v[i], q2 + q2), q2), q);
    __syncthreads();
    row8_fwd_tail<S, EPI>(a, srow, lr, r, t, poly);
  } else {
    const u64* in = a.src + limb_src_off(a, blockIdx.y, lr) + (size_t)r * C;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = __builtin_nontemporal_load(&in[w8_elem(L0, t, i)]);
#pragma unroll
    for (int i = 0; i < 8; i++) srow[w8_swz(w8_elem(L0, t, i))] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = srow[w8_swz(w8_elem(LL, t, i))];
#pragma unroll
    for (int k = NR - 1; k >= 0; k--) {
      if (k < NR - 1) {
        const int lp = w8_ls(S, k + 1), lc = w8_ls(S, k);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) srow[w8_swz(w8_elem(lp, t, i))] = v[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = srow[w8_swz(w8_elem(lc, t, i))];
      }
      if (k == 2) w8_round<false, S, 2>(v, t, A, 0, Nn, tw, q);
      if (k == 1) w8_round<false, S, 1>(v, t, A, 0, Nn, tw, q);
      if (k == 0) w8_round<false, S, 0>(v, t, A, 0, Nn, tw, q);
    }
    // the last round is round 0: its order is the coalesced one
#pragma unroll
    for (int i = 0; i < 8; i++) __builtin_nontemporal_store(v[i], &poly[w8_elem(L0, t, i)]);
  }
}
template <bool FWD, int S, bool EPI>
__device__ __forceinline__ void ntt_row8_fp(const NttArgs& a, u64* sm, const LimbRef& lr) {
  constexpr int T = 1 << (S - 3), C = 1 << S, NR = (S + 2) / 3;
  constexpr int L0 = w8_ls(S, 0), LL = w8_ls(S, NR - 1);
  static_assert(FWD ? fpb::ct_pass_ok(true, S, false) : fpb::gs_pass_ok(true, S, true),
                "float64 8-word row pass out of bounds");
  const int tid = threadIdx.x;
  const int t = tid & (T - 1);
  const int rho = tid >> (S - 3);
  const int m = lr.mod;
  const FpC fc = a.fpc[m];
  const u64 Nn = 1ull << a.logN;
  const int r = blockIdx.x * a.nsub + rho;
  u64* poly = a.data + lr.off + (size_t)r * C;
  u64* srow = sm + rho * C;
  const uint4* tw = a.tw + (size_t)m * Nn;
  const u64 A = (u64)r * C;
  double v[8];
  if (FWD) {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = f_val(__builtin_nontemporal_load(&poly[w8_elem(L0, t, i)]));
    w8_round_fp<true, S, 0, false>(v, t, A, 0, Nn, tw, fc);
#pragma unroll
    for (int k = 1; k < NR; k++) {
      const int lp = w8_ls(S, k - 1), lc = w8_ls(S, k);
      if (k > 1) __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) srow[w8_swz(w8_elem(lp, t, i))] = f_bits(v[i]);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = f_val(srow[w8_swz(w8_elem(lc, t, i))]);
      if (k == 1) w8_round_fp<true, S, 1, false>(v, t, A, 0, Nn, tw, fc);
      if (k == 2) w8_round_fp<true, S, 2, false>(v, t, A, 0, Nn, tw, fc);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) srow[w8_swz(w8_elem(LL, t, i))] = f_canon(v[i], fc);
    __syncthreads();
    row8_fwd_tail<S, EPI>(a, srow, lr, r, t, poly);
  } else {
    const u64* in = a.src + limb_src_off(a, blockIdx.y, lr) + (size_t)r * C;
    u64 w[8];
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = __builtin_nontemporal_load(&in[w8_elem(L0, t, i)]);
#pragma unroll
    for (int i = 0; i < 8; i++) srow[w8_swz(w8_elem(L0, t, i))] = w[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = f_in(srow[w8_swz(w8_elem(LL, t, i))]);
#pragma unroll
    for (int k = NR - 1; k >= 0; k--) {
      if (k < NR - 1) {
        const int lp = w8_ls(S, k + 1), lc = w8_ls(S, k);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) srow[w8_swz(w8_elem(lp, t, i))] = f_bits(v[i]);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = f_val(srow[w8_swz(w8_elem(lc, t, i))]);
      }
      if (k == 2) w8_round_fp<false, S, 2, true>(v, t, A, 0, Nn, tw, fc);
      if (k == 1) w8_round_fp<false, S, 1, true>(v, t, A, 0, Nn, tw, fc);
      if (k == 0) w8_round_fp<false, S, 0, true>(v, t, A, 0, Nn, tw, fc);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) __builtin_nontemporal_store(f_bits(v[i]), &poly[w8_elem(L0, t, i)]);
  }
}
template <bool FWD, int S, bool EPI = false>
__global__ __launch_bounds__(256) void ntt_row8_kernel(NttArgs a) {
  __shared__ u64 sm[2048];
  const LimbRef lr = limb_ref(a, blockIdx.y);
  if (a.mods[lr.mod].q <= FP_QMAX) ntt_row8_fp<FWD, S, EPI>(a, sm, lr);
  else ntt_row8_int<FWD, S, EPI>(a, sm, lr);
}

template <bool FWD>
void launch_col(int S, dim3 grid, dim3 block, const NttArgs& a, hipStream_t st) {
  switch (S) {
    case 5: hipLaunchKernelGGL((ntt_col_kernel<FWD, 5>), grid, block, 0, st, a); break;
    case 6: hipLaunchKernelGGL((ntt_col_kernel<FWD, 6>), grid, block, 0, st, a); break;
    case 7: hipLaunchKernelGGL((ntt_col_kernel<FWD, 7>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((ntt_col_kernel<FWD, 8>), grid, block, 0, st, a); break;
  }
}
// The ModDown epilogue is its own instantiation so that the plain forward
// pass keeps its smaller register footprint (and occupancy).
template <bool FWD, bool EPI>
void launch_row_t(int S, dim3 grid, dim3 block, const NttArgs& a, hipStream_t st) {
  switch (S) {
    case 5: hipLaunchKernelGGL((ntt_row_kernel<FWD, 5, EPI>), grid, block, 0, st, a); break;
    case 6: hipLaunchKernelGGL((ntt_row_kernel<FWD, 6, EPI>), grid, block, 0, st, a); break;
    case 7: hipLaunchKernelGGL((ntt_row_kernel<FWD, 7, EPI>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((ntt_row_kernel<FWD, 8, EPI>), grid, block, 0, st, a); break;
  }
}
template <bool FWD>
void launch_row(int S, dim3 grid, dim3 block, const NttArgs& a, hipStream_t st) {
  if (FWD && a.epi) launch_row_t<true, true>(S, grid, block, a, st);
  else launch_row_t<FWD, false>(S, grid, block, a, st);
}
template <bool FWD>
void launch_col8(int S, dim3 grid, dim3 block, const NttArgs& a, hipStream_t st) {
  switch (S) {
    case 5: hipLaunchKernelGGL((ntt_col8_kernel<FWD, 5>), grid, block, 0, st, a); break;
    case 6: hipLaunchKernelGGL((ntt_col8_kernel<FWD, 6>), grid, block, 0, st, a); break;
    case 7: hipLaunchKernelGGL((ntt_col8_kernel<FWD, 7>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((ntt_col8_kernel<FWD, 8>), grid, block, 0, st, a); break;
  }
}
template <bool FWD, bool EPI>
void launch_row8_t(int S, dim3 grid, dim3 block, const NttArgs& a, hipStream_t st) {
  switch (S) {
    case 5: hipLaunchKernelGGL((ntt_row8_kernel<FWD, 5, EPI>), grid, block, 0, st, a); break;
    case 6: hipLaunchKernelGGL((ntt_row8_kernel<FWD, 6, EPI>), grid, block, 0, st, a); break;
    case 7: hipLaunchKernelGGL((ntt_row8_kernel<FWD, 7, EPI>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((ntt_row8_kernel<FWD, 8, EPI>), grid, block, 0, st, a); break;
  }
}
template <bool FWD>
void launch_row8(int S, dim3 grid, dim3 block, const NttArgs& a, hipStream_t st) {
  if (FWD && a.epi) launch_row8_t<true, true>(S, grid, block, a, st);
  else launch_row8_t<FWD, false>(S, grid, block, a, st);
}

}  // namespace

int ntt_row_round_slots(int logN) {
  int SA, SB;
  ntt_split(logN, &SA, &SB);
  return ntt_round_slots(SB - 4);
}

// Split of logN into column (SA) and row (SB) sub-transform sizes.
void ntt_split(int logN, int* SA, int* SB) {
  *SA = logN / 2;
  *SB = logN - *SA;
}

void launch_ntt(u64* data, size_t bstride, int batch, RowMap rm, int logN, bool forward, const NttTables& tw,
                hipStream_t st) {
  launch_ntt(data, bstride, data, bstride, batch, rm, logN, forward, tw, st);
}

// Workgroup shape: 256-thread tiles (narrower tiles lose coalescing and
// measured slower even for launches of a few limbs).
// Launches over at most this many limbs use the 8-word kernels (a launch of
// few limbs leaves most SIMDs with one or two waves of the 16-word kernels).
#ifndef NTT_W8_MAX_LIMBS
#define NTT_W8_MAX_LIMBS 96
#endif

static void ntt_launch(NttArgs a, int nlimbs, bool forward, hipStream_t st) {
  int SA, SB;
  ntt_split(a.logN, &SA, &SB);
  a.SA = SA; a.SB = SB;
  if (nlimbs <= NTT_W8_MAX_LIMBS) {
    const int TA = 1 << (SA - 3), TB = 1 << (SB - 3), C = 1 << SB, R = 1 << SA;
    const int nsubA = std::min(512 / TA, C), nsubB = std::min(256 / TB, R);
    NttArgs aA = a; aA.nsub = nsubA;
    NttArgs aB = a; aB.nsub = nsubB;
    if (forward) { aB.src = a.data; aB.sstride = a.bstride; } else { aA.src = a.data; aA.sstride = a.bstride; }
    dim3 gridA(C / nsubA, nlimbs), blockA(TA * nsubA);
    dim3 gridB(R / nsubB, nlimbs), blockB(TB * nsubB);
    if (forward) {
      launch_col8<true>(SA, gridA, blockA, aA, st);
      launch_row8<true>(SB, gridB, blockB, aB, st);
    } else {
      launch_row8<false>(SB, gridB, blockB, aB, st);
      launch_col8<false>(SA, gridA, blockA, aA, st);
    }
    return;
  }
  const int PA = 1 << (SA - 4), C = 1 << SB, R = 1 << SA;
  const int PB = 1 << (SB - 4);
  const int nsubA = std::min(NTT_TPB / PA, C), nsubB = std::min(NTT_TPB / PB, R);
  NttArgs aA = a; aA.nsub = nsubA;
  NttArgs aB = a; aB.nsub = nsubB;
  // only the first pass reads src
  if (forward) { aB.src = a.data; aB.sstride = a.bstride; } else { aA.src = a.data; aA.sstride = a.bstride; }
  dim3 gridA(C / nsubA, nlimbs), blockA(PA * nsubA);
  dim3 gridB(R / nsubB, nlimbs), blockB(PB * nsubB);
  if (forward) {
    launch_col<true>(SA, gridA, blockA, aA, st);
    launch_row<true>(SB, gridB, blockB, aB, st);
  } else {
    launch_row<false>(SB, gridB, blockB, aB, st);
    launch_col<false>(SA, gridA, blockA, aA, st);
  }
}

void launch_ntt(const u64* src, size_t sstride, u64* data, size_t bstride, int batch, RowMap rm, int logN, bool forward,
                const NttTables& tw, hipStream_t st) {
  const int rows = rm.nact();
  if (rows <= 0 || batch <= 0) return;
  NttArgs a{};
  a.list = nullptr;
  a.src = src; a.sstride = sstride; a.data = data; a.bstride = bstride; a.rm = rm; a.rows = rows; a.batch = batch;
  a.mods = tw.mods;
  a.ninv = tw.ninv; a.ninvp = tw.ninvp; a.fpc = tw.fpc; a.logN = logN;
  a.tw = reinterpret_cast<const uint4*>(forward ? tw.tw : tw.itw);
  a.twr = reinterpret_cast<const uint4*>(forward ? tw.twr : tw.itwr);
  ntt_launch(a, rows * batch, forward, st);
}

void launch_ntt_moddown(u64* ext, size_t ext_bstride, int batch, int l, int logN, const u64* x, size_t x_bstride,
                        u64* out, size_t o_bstride, const u64* add, size_t a_bstride, int add_batches,
                        const uint32_t* perm_inv, const u64* pinv, const u64* pinvp, const NttTables& tw, hipStream_t st,
                        const u64* acc, size_t c_bstride) {
  const RowMap rm{l + 1, l + 1, 0, 0, 0, 0};
  NttArgs a{};
  a.list = nullptr;
  a.src = ext; a.sstride = ext_bstride; a.data = ext; a.bstride = ext_bstride; a.rm = rm; a.rows = l + 1; a.batch = batch;
  a.mods = tw.mods;
  a.ninv = tw.ninv; a.ninvp = tw.ninvp; a.fpc = tw.fpc; a.logN = logN;
  a.tw = reinterpret_cast<const uint4*>(tw.tw);
  a.twr = reinterpret_cast<const uint4*>(tw.twr);
  a.epi = 1;
  a.e = ModDownEpi{x, x_bstride, out, o_bstride, add, a_bstride, add_batches, perm_inv, pinv, pinvp, acc, c_bstride,
                   nullptr, 0, nullptr};
  ntt_launch(a, (l + 1) * batch, true, st);
}
void launch_ntt_rescale_pair(u64* t, size_t t_bstride, int l, int logN, const u64* x, size_t x_bstride, u64* out0,
                             u64* out1, size_t o_bstride, const u64* ks, const u64* rsinv, const u64* rsinvp,
                             const NttTables& tw, hipStream_t st) {
  const RowMap rm{l, l, 0, 0, 0, 0};
  NttArgs a{};
  a.list = nullptr;
  a.src = t; a.sstride = t_bstride; a.data = t; a.bstride = t_bstride; a.rm = rm; a.rows = l; a.batch = 4;
  a.mods = tw.mods;
  a.ninv = tw.ninv; a.ninvp = tw.ninvp; a.fpc = tw.fpc; a.logN = logN;
  a.tw = reinterpret_cast<const uint4*>(tw.tw);
  a.twr = reinterpret_cast<const uint4*>(tw.twr);
  a.epi = 1;
  a.e = ModDownEpi{x, x_bstride, out0, o_bstride, nullptr, 0, 0, nullptr, rsinv, rsinvp, nullptr, 0, ks, l, out1};
  ntt_launch(a, l * 4, true, st);
}

void launch_ntt_list(u64* data, const void* list, int nlimbs, int logN, bool forward, const NttTables& tw, hipStream_t st) {
  if (nlimbs <= 0) return;
  NttArgs a{};
  a.list = reinterpret_cast<const LimbRef*>(list);
  a.src = data; a.data = data; a.mods = tw.mods; a.rows = 1; a.batch = 1;
  a.ninv = tw.ninv; a.ninvp = tw.ninvp; a.fpc = tw.fpc; a.logN = logN;
  a.tw = reinterpret_cast<const uint4*>(forward ? tw.tw : tw.itw);
  a.twr = reinterpret_cast<const uint4*>(forward ? tw.twr : tw.itwr);
  ntt_launch(a, nlimbs, forward, st);
}
