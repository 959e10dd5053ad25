/*
 * ckks_oracle.h -- CPU restatement of the CKKS arithmetic on the HE-LRM
 * embedding-PCMM path, used ONLY as the checker (tests, smoke(), and the
 * cpu_baseline leg of bench.py).  It is test infrastructure, not product
 * code: nothing under helrm_amd/ links, loads or calls it.
 *
 * What it restates.  The reference evaluates the PCMM through Orion's
 * Lattigo backend (the Go files of orion/backend/lattigo), a cgo wrapper over the
 * un-vendored Go module github.com/baahl-nyu/lattigo/v6 v6.2.0
 * (orion/backend/lattigo/go.mod:6).  That module is absent from the
 * reference tree, so each function below restates the published Lattigo
 * v6 algorithm it stands for, anchored on the wrapper call sites:
 *   scheme / keys      scheme.go:35-87, keygenerator.go:13-35, evaluator.go:29-66
 *   encode / decode    encoder.go:16-48      (values cross as C.float)
 *   encrypt / decrypt  encryptor.go:20-38
 *   rotate / rescale   evaluator.go:90-146
 *   add                evaluator.go:229-235, 298-304
 *   linear transform   lineartransform.go:36-128
 *
 * Conventions (shared with the product so raw buffers compare directly):
 *   - polynomials are limb-major arrays u64[limbs][N];
 *   - the NTT domain is the negacyclic evaluation at psi^(2*brv(j)+1) in
 *     slot j (bit-reversed order), psi = g^((q-1)/2N), g the smallest
 *     generator of Z_q^*;
 *   - a QP polynomial at level l holds limbs q_0..q_l then p_0..p_{K-1};
 *   - key material and encryption randomness come from the counter PRNG
 *     described in ckks_oracle.c (own construction, documented there).
 *
 * Parity status per function is recorded in the header comment of
 * ckks_oracle.c.
 */
#ifndef CKKS_ORACLE_H
#define CKKS_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_ctx orc_ctx;
typedef struct orc_lt orc_lt;

/* ---- number theory / primitives ------------------------------------ */
int      orc_is_prime(uint64_t n);
int      orc_gen_primes(int logN, const int* logq, int nq, const int* logp,
                        int np, uint64_t* q_out, uint64_t* p_out);
uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q);
uint64_t orc_rand64(uint64_t seed, uint64_t stream, uint64_t ctr);

/* ---- context --------------------------------------------------------- */
orc_ctx* orc_new(int logN, const uint64_t* q, int L, const uint64_t* p, int K,
                 int h, uint64_t seed);
void     orc_free(orc_ctx* c);
int      orc_N(const orc_ctx* c);
uint64_t orc_modulus(const orc_ctx* c, int idx); /* idx < L: q, else p */
uint64_t orc_galois_element(const orc_ctx* c, int k);
void     orc_ntt(const orc_ctx* c, int mod_idx, uint64_t* a);
void     orc_intt(const orc_ctx* c, int mod_idx, uint64_t* a);
void     orc_automorphism_index(const orc_ctx* c, uint64_t galel, uint32_t* idx);

/* ---- keys ------------------------------------------------------------- */
void orc_secret_key(const orc_ctx* c, int64_t* s_coeffs);
/* Galois key [dnum][2][L+K][N] in the NTT domain (cached in the context). */
const uint64_t* orc_galois_key(orc_ctx* c, uint64_t galel);
void orc_public_key(const orc_ctx* c, uint64_t* out); /* [2][L+K][N] */
/* Relinearization key (s^2 -> s) [dnum][2][L+K][N], NTT (cached). */
const uint64_t* orc_relin_key(orc_ctx* c);

/* ---- encoder ----------------------------------------------------------- */
void orc_encode(const orc_ctx* c, const float* v, int n, int level,
                double scale, int with_p, uint64_t* out);
void orc_encode_f64(const orc_ctx* c, const double* v, int n, int level,
                    double scale, int with_p, uint64_t* out);
void orc_decode(const orc_ctx* c, const uint64_t* pt, int level, double scale,
                float* out);
void orc_decode_f64(const orc_ctx* c, const uint64_t* pt, int level,
                    double scale, double* out);

/* ---- encryptor --------------------------------------------------------- */
void orc_encrypt(const orc_ctx* c, const uint64_t* pt, int level,
                 uint64_t enc_index, uint64_t* ct);
void orc_encode_complex_f64(const orc_ctx* c, const double* v, const double* vi, int n, int level, double scale, int with_p,
                            uint64_t* out);
void orc_encode_complex(const orc_ctx* c, const float* v, int n, int level, double scale, uint64_t* out);
void orc_decode_complex_f64(const orc_ctx* c, const uint64_t* pt, int level, double scale, double* out);
void orc_mul_i(const orc_ctx* c, const uint64_t* ct, int l, int npoly, uint64_t* out);
void orc_expand_seeded_a(const orc_ctx* c, int l, uint64_t seed, uint64_t* a);
void orc_encrypt_seeded(const orc_ctx* c, const uint64_t* pt, int l, uint64_t seed, uint64_t enc, uint64_t* ct);
void orc_decrypt(const orc_ctx* c, const uint64_t* ct, int level, uint64_t* pt);

/* ---- plaintext / scalar / ciphertext products ----------------------------- */
void orc_mul_plain(const orc_ctx* c, const uint64_t* ct, int lc, const uint64_t* pt, int lp, uint64_t* out);
int  orc_scaled_constant(double v, double scale, int64_t* out);
void orc_mul_int(const orc_ctx* c, const uint64_t* ct, int l, int64_t k, uint64_t* out);
int  orc_mul_float(const orc_ctx* c, const uint64_t* ct, int l, double v, uint64_t* out);
int  orc_add_const(const orc_ctx* c, const uint64_t* ct, int l, double v, double scale, int sub, uint64_t* out);
void orc_mul_relin(orc_ctx* c, const uint64_t* a, const uint64_t* b, int l, uint64_t* out);
/* Monomial polynomial of degree <= 3 on a ciphertext at level l and scale s;
 * returns the output level (output scale = so), -1 if unsupported. */
int  orc_eval_poly(orc_ctx* c, const uint64_t* x, int l, double s, const double* coef, int d, double so, uint64_t* out);

/* ---- evaluator --------------------------------------------------------- */
void orc_add(const orc_ctx* c, const uint64_t* a, const uint64_t* b, int level,
             int npoly, uint64_t* out);
void orc_rescale(const orc_ctx* c, const uint64_t* ct, int level, uint64_t* out);
void orc_rotate(orc_ctx* c, const uint64_t* ct, int level, int k, uint64_t* out);
void orc_automorphism_ct(orc_ctx* c, const uint64_t* ct, int level,
                         uint64_t galel, uint64_t* out);
void orc_mod_down(const orc_ctx* c, int level, const uint64_t* qp, uint64_t* q_out);
void orc_decompose_modup(const orc_ctx* c, int level, const uint64_t* c1_ntt,
                         uint64_t* digits);
void orc_basis_extend(const orc_ctx* c, const int* src, int ns, const int* dst,
                      int nd, const uint64_t* in, uint64_t* out);

/* ---- linear transform (BSGS diagonal evaluation) ------------------------ */
orc_lt* orc_lt_new(orc_ctx* c, const int* idx, int nidx, const float* data,
                   int level, float bsgs_ratio);
void    orc_lt_free(orc_lt* t);
int     orc_lt_n1(const orc_lt* t);
int     orc_lt_level(const orc_lt* t);
int     orc_lt_num_plaintexts(const orc_lt* t);
int     orc_lt_plaintext_index(const orc_lt* t, int i);
const uint64_t* orc_lt_plaintext(const orc_lt* t, int diag_index);
int     orc_lt_rotations(const orc_lt* t, int* out);
void    orc_lt_eval(orc_ctx* c, const orc_lt* t, const uint64_t* ct,
                    int ct_level, uint64_t* out);
int     orc_lt_num_giant(const orc_lt* t);
void    orc_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
