// kernels.h -- launch interface of kernels.hip (internal to the library).
#pragma once
#include "hipckks.h"

// Per-modulus constants of the float64 transform (moduli q <= FP_QMAX,
// fpntt.h); the other moduli leave the entry unused.
struct FpC {
  double q, qinv;  // q and fl(1/q)
  double cneg;     // 2^52 + q (canonical output of a negative residue)
  double ni, niq;  // N^-1 centred, and fl(N^-1 / q)
  double wn, wnq;  // the inverse transform's last twiddle times N^-1, centred, and fl(wn / q)
  double pad;
};
struct NttTables {
  const ModC* mods;
  // [mod][N][2]: (psi^brv(k), Shoup companion) and the same for psi^-1; for
  // a modulus q <= FP_QMAX the pair is (w, fl(w / q)) as float64 bits with
  // w = psi^brv(k) centred in (-q/2, q/2]
  const u64 *tw, *itw;
  const u64 *twr, *itwr;   // [mod][R][slots][P][2]: row-pass consecutive-round twiddles, lane-interleaved
  const u64 *ninv, *ninvp; // [mod]
  const FpC* fpc;          // [mod]
};
// N = R x C, R = 2^SA, C = 2^SB (the transform's column / row split)
void ntt_split(int logN, int* SA, int* SB);
// twiddle slots per lane of the row pass's consecutive round
int ntt_row_round_slots(int logN);

struct BConvSrc {
  u64 q, hinv, hinvp;  // source modulus, (S/s_i)^-1 mod s_i and its Shoup companion
  double qd;           // (double)q
};
struct BConvTable {
  BConvSrc src[HCK_MAXSRC];
  const u64* hat;  // [nmod][ns]   (S/s_i mod t) * R mod t  (Montgomery form)
  const u64* vS;   // [nmod][ns+1] v*S mod t
  int rows_per_block;
};

struct KeyMacArgs {
  const u64* digits;       // [dn][nqp][N] (per batch if digits_per_batch)
  size_t dig_bstride;
  int digits_per_batch;
  const u64* const* key;   // per batch: [dnum][2][L+K][N] Montgomery form (nullptr: use key1)
  const uint32_t* const* perm;  // per batch (nullptr: use perm1)
  const u64* key1;         // single-batch key
  const uint32_t* perm1;   // single-batch permutation (nullptr: identity)
  const u64* add0;         // Q rows added to part 0 before the gather (mode 1)
  const u64* own;          // the decomposed polynomial (NTT, Q rows; per batch if digits_per_batch): a
  size_t own_bstride;      // digit's own rows are read from it (nullptr: from the digit buffer)
  u64 *out0, *out1;
  size_t out_bstride;
  const ModC* mods;
  int N, l, L, K, nqp, dn;
};

struct GiantAccArgs {
  const u64* digits;  // [ng][dn][nqp][N]
  size_t dig_bstride;
  const u64* const* key;       // [ng]
  const uint32_t* const* perm; // [ng]
  const int* tg;               // giant-group index into T per key-switched group
  int ng;
  const u64* own;              // [ng][l+1][N] decomposed polynomials (own digit rows), or nullptr
  size_t own_bstride;
  const u64* T;                // [ngroups][2][nqp][N]
  size_t T_gstride, T_pstride;
  int t_zero;                  // index of the rotation-0 group in T, or -1
  u64 *out0, *out1;            // QP accumulators [nqp][N]
  const ModC* mods;
  int N, l, L, K, nqp, dn;
};

struct DiagMacArgs {
  const u64* diag;        // [np][lt_level+1+K][N] Montgomery form
  size_t diag_stride;
  const u64* pc;          // P*c0, P*c1 : [2][l+1][N]
  size_t pc_pstride;
  const int* baby_is_zero;  // [nbaby]
  const int* baby_slot;     // [nbaby]
  const int* gpi;           // [ng][nbaby] plaintext index of baby b in group g (absent: a zero plaintext)
  int dense;                // every group holds every baby: index = g * nbaby + b
  int zero_pidx;            // index of the all-zero plaintext (babies past nbaby in a chunk use it)
  u64* T;                   // [ng][2][nqp][N]
  size_t T_gstride, T_pstride;
  const ModC* mods;
  int N, l, L, K, nqp, lt_level, ng, nbaby, b0, nb_chunk;
  int g0, g1;               // giant groups [g0, g1) of this launch
  // the hoisted baby rotations, computed in the kernel's prologue
  // (keymac_kernel's arithmetic per word)
  const u64* digits;              // [dn][nqp][N] decomposition of c1 (NTT)
  const u64* const* bkey;         // per baby slot: Galois key [dnum][2][L+K][N], Montgomery form
  const uint32_t* const* bperm;   // per baby slot: automorphism gather
  const u64* own;                 // c1 (Q rows, NTT): a digit's own rows
  int dn;
};

// In-place NTT (forward) / inverse NTT of rows rm of `batch` polynomials.
void launch_ntt(u64* data, size_t bstride, int batch, RowMap rm, int logN, bool forward, const NttTables& tw, hipStream_t st);
// Out-of-place: the transform of src's rows is written to the same rows of dst.
void launch_ntt(const u64* src, size_t sstride, u64* dst, size_t dstride, int batch, RowMap rm, int logN, bool forward,
                const NttTables& tw, hipStream_t st);
// In-place NTT / inverse NTT of an explicit list of limbs: list is a device
// array of nlimbs {int64 word offset from data, int modulus index, int pad}.
void launch_ntt_list(u64* data, const void* list, int nlimbs, int logN, bool forward, const NttTables& tw, hipStream_t st);
// Forward NTT of the Q rows 0..l of ext (the extension of [x]_P to Q) fused
// with the ModDown combine: out[b][i][perm_inv^-1...] -- for every position p,
// out[b][i][perm_inv[p]] = (x[b][i][p] - NTT(ext)[b][i][p]) * P^-1 (+ add[b][i][p]
// for b < add_batches) (+ acc[b][i][perm_inv[p]] if acc, a buffer other than
// out); ext itself is left in an intermediate state.
void launch_ntt_moddown(u64* ext, size_t ext_bstride, int batch, int l, int logN, const u64* x, size_t x_bstride,
                        u64* out, size_t o_bstride, const u64* add, size_t a_bstride, int add_batches,
                        const uint32_t* perm_inv, const u64* pinv, const u64* pinvp, const NttTables& tw, hipStream_t st,
                        const u64* acc = nullptr, size_t c_bstride = 0);
// dst[b][0..words) = src[b][0..words) for b < batch.
void launch_copy(u64* dst, size_t dstride, const u64* src, size_t sstride, size_t words, int batch, hipStream_t st);
void launch_add(u64* out, const u64* a, const u64* b, size_t bstride, int batch, RowMap rm, const ModC* mods, int N, bool sub, hipStream_t st);
void launch_mul_const(u64* out, const u64* in, size_t bstride, int batch, RowMap rm, const u64* cw, const u64* cwp, const ModC* mods, int N, hipStream_t st);
void launch_mont_mul(u64* out, size_t obstride, const u64* a, size_t abstride, const u64* bR, size_t bbstride, int batch, RowMap rm, const ModC* mods, int N, bool acc, hipStream_t st);
void launch_mont_convert(u64* data, size_t bstride, int batch, RowMap rm, const ModC* mods, int N, bool to, hipStream_t st);
// out = in +- c[modulus] on the rows of rm (one polynomial)
void launch_add_scalar(u64* out, const u64* in, RowMap rm, const u64* c, const ModC* mods, int N, bool sub, hipStream_t st);
// Basis extension of the ns source rows of `in` into the target rows rm of `out`.
// One source group of a batched basis extension (e.g. one digit of a
// decomposition): its table (device copy), source rows, destination rows.
struct BConvJob {
  const BConvTable* tab;
  int src_row, ns, force_v0, pad;
  RowMap rm;
  size_t out_off;  // word offset of the group's output inside a batch entry
};
#define HCK_MAXJOBS 16
struct BConvJobs { BConvJob j[HCK_MAXJOBS]; int n, rows_per_block; };
// Basis extension of every job for every batch entry, in one launch.
void launch_bconv(const u64* in, size_t in_bstride, BConvJobs jobs, u64* out, size_t out_bstride, int batch,
                  const ModC* mods, int N, hipStream_t st);
// Single source group: the sources are rows [0, ns) of in.
void launch_bconv(const u64* in, size_t in_bstride, int ns, const BConvTable* dtab, u64* out, size_t out_bstride, int batch,
                  const RowMap& rm, const ModC* mods, int N, bool force_v0, hipStream_t st);
void launch_moddown_combine(u64* out, size_t o_bstride, const u64* x, size_t x_bstride, const u64* ext, size_t e_bstride, const u64* add, size_t a_bstride, int add_batches, const uint32_t* perm, const u64* pinv, const u64* pinvp, int qrows, int batch, const ModC* mods, int N, hipStream_t st);
void launch_keymac(const KeyMacArgs& a, int batch, hipStream_t st);
void launch_giant_acc(const GiantAccArgs& a, hipStream_t st);
void launch_diag_mac(const DiagMacArgs& a, hipStream_t st);
void launch_rescale_spread(u64* t, const u64* u, int l, u64 half, const ModC* mods, int N, hipStream_t st);
// ModDown + rescale: rows i < l of the coefficient-domain extension ext become
// ext_i + P * t_i, t the rescale's spread of the ModDown result's row l
// ((xl - ext_l) * P^-1 mod q_l); ext and xl have `batch` entries.
void launch_moddown_rescale_spread(u64* ext, size_t e_bstride, const u64* xl, size_t x_bstride, int l, u64 half, u64 pinvl,
                                   u64 pinvlp, const u64* pmod_w, const u64* pmod_wp, const ModC* mods, int N, int batch,
                                   hipStream_t st);
void launch_sample_uniform(u64* out, RowMap rm, u64 seed, u64 stream, const ModC* mods, int N, hipStream_t st);
void launch_sample_cbd(u64* out, RowMap rm, u64 seed, u64 stream, const ModC* mods, int N, bool add, hipStream_t st);
void launch_signed_rows(u64* out, RowMap rm, const int8_t* v, const ModC* mods, int N, hipStream_t st);
void launch_gk_combine(u64* b, const u64* a, const u64* soR, const u64* sR, int own0, int own1, const u64* pmod, int rows, const ModC* mods, int N, hipStream_t st);
// Device encoder (encoder.hip): plaintext p of a batch takes element k from
// data[src * slots + ((k + rot) mod slots)] (zero past nvals), runs the special
// inverse FFT in float64 (work buffers re/im, pstride words per plaintext),
// rounds to fixed point at `scale` and writes its residues to rows rm of
// out + p * out_pstride (coefficient domain; the caller applies the NTT).
struct EncodeSrc { int src, rot; };
void launch_encode_fft(u64* out, size_t out_pstride, RowMap rm, const float* data, const EncodeSrc* src, int np, int nvals,
                       double scale, double* re, double* im, size_t pstride, const int* rotgroup, const double* rre,
                       const double* rim, const ModC* mods, int logN, hipStream_t st, bool complex_in = false);
// multiplication by the imaginary unit (the monomial X^(N/2)) in the NTT domain:
// slot x < N/2 times iu[m], slot x >= N/2 times q - iu[m] (Shoup pairs iu / iup, niu / niup)
void launch_mul_i(u64* out, const u64* in, size_t bstride, int batch, RowMap rm, const u64* iu, const u64* iup,
                  const u64* niu, const u64* niup, const ModC* mods, int N, hipStream_t st);
// out[r][x] = sum_{p < npoly} a[p][r][x] * b[p][r][x] mod q_r, rows r < nrows of the modulus table
void launch_mulacc(const u64* a, const u64* b, u64* out, int npoly, int nrows, const ModC* mods, int N, hipStream_t st);
// Integer VALU issue-rate probe: `blocks` workgroups of 256 lanes, each lane
// iters x 8 independent instructions (op 0: v_mad_u64_u32, op 1: v_add3_u32);
// one word per lane written to out.
void launch_valu_probe(int op, u64* out, int blocks, uint32_t seed, int iters, hipStream_t st);
