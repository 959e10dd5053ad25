/*
 * ckks_oracle.c -- CPU restatement (checker only) of the CKKS arithmetic
 * that the reference runs for the HE-LRM embedding PCMM through Orion's
 * Lattigo backend.  TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load this library, always as the checker.
 *
 * The algorithms live in the un-vendored Go module
 * github.com/baahl-nyu/lattigo/v6 v6.2.0 (orion/backend/lattigo/go.mod:6).
 * Each function restates the published Lattigo v6 algorithm named in its
 * comment and cites the wrapper call site in the reference that reaches it.
 *
 * Parity pins (tests/test_oracle_*.py):
 *   orc_ntt / orc_intt        schoolbook negacyclic product + direct
 *                             evaluation at psi^(2 brv(j)+1)       PINNED
 *   orc_basis_extend          exact big-integer CRT at small N      PINNED
 *   orc_mod_down              (x - [x]_P)/P big-integer identity     PINNED
 *   orc_rescale               round(x / q_l) big-integer identity    PINNED
 *   orc_encode / orc_decode   direct O(N^2) canonical embedding      PINNED
 *   orc_encrypt / decrypt     decrypt(encrypt(m)) - m within noise   PINNED
 *   orc_rotate                decoded slot rotation (closed form)    PINNED
 *   orc_lt_*                  identity / shift / multi-diagonal
 *                             closed forms (test_linear_transform.py)
 *                             and dense mat-vec on random diagonals PINNED
 *   orc_gen_primes            primality + p = 1 mod 2N + bit size   PINNED
 *   Lattigo-internal choices that only the Go module itself could pin
 *   (the order of its prime generator, Go's math.Cos in the FFT roots,
 *   its PRNG and samplers) are restated from the published algorithm and
 *   recorded as "parity unpinned against Lattigo" in the design notes.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include "ckks_oracle.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef uint64_t u64;
typedef int64_t i64;
typedef unsigned __int128 u128;

#define MAXMOD 96
#define BIGW 80 /* big-integer words (80*64 = 5120 bits) */

static void die(const char* m) { fprintf(stderr, "oracle: %s\n", m); abort(); }
static void* xmalloc(size_t n) { void* p = malloc(n ? n : 1); if (!p) die("out of memory"); return p; }
static void* xcalloc(size_t n) { void* p = calloc(1, n ? n : 1); if (!p) die("out of memory"); return p; }

/* =====================================================================
 * 1. Modular arithmetic (q < 2^62)
 * ===================================================================== */
typedef struct { u64 q, mu; int b; } barrett_t; /* HAC 14.42, mu = floor(2^2b / q) */

static barrett_t barrett_make(u64 q) {
    barrett_t r; r.q = q; r.b = 64 - __builtin_clzll(q);
    r.mu = (u64)(((u128)1 << (2 * r.b)) / q);
    return r;
}
static inline u64 barrett_reduce(const barrett_t* B, u128 x) { /* x < q^2 */
    u64 x1 = (u64)(x >> (B->b - 1));
    u64 t = (u64)(((u128)x1 * B->mu) >> (B->b + 1));
    u64 r = (u64)x - t * B->q;
    while (r >= B->q) r -= B->q;
    return r;
}
static inline u64 mulmod_b(const barrett_t* B, u64 a, u64 b) { return barrett_reduce(B, (u128)a * b); }
static inline u64 addmod(u64 a, u64 b, u64 q) { u64 r = a + b; return r >= q ? r - q : r; }
static inline u64 submod(u64 a, u64 b, u64 q) { return a >= b ? a - b : a + q - b; }
static inline u64 negmod(u64 a, u64 q) { return a ? q - a : 0; }

uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q) { return (u64)(((u128)a * b) % q); }

static u64 powmod(u64 a, u64 e, u64 q) {
    u64 r = 1 % q; a %= q;
    while (e) { if (e & 1) r = orc_mulmod(r, a, q); a = orc_mulmod(a, a, q); e >>= 1; }
    return r;
}
static u64 invmod_prime(u64 a, u64 q) { return powmod(a % q, q - 2, q); }
static u64 invmod_generic(u64 a, u64 m) { /* extended Euclid, gcd(a,m)=1 */
    i64 t = 0, nt = 1; u64 r = m, nr = a % m;
    while (nr) { u64 qq = r / nr; i64 tmp = t - (i64)qq * nt; t = nt; nt = tmp; u64 tr = r - qq * nr; r = nr; nr = tr; }
    if (t < 0) t += (i64)m;
    return (u64)t;
}
static inline u64 shoup_pre(u64 w, u64 q) { return (u64)(((u128)w << 64) / q); }
static inline u64 shoup_mul(u64 x, u64 w, u64 wp, u64 q) {
    u64 qh = (u64)(((u128)x * wp) >> 64);
    u64 r = x * w - qh * q;
    return r >= q ? r - q : r;
}

/* Deterministic Miller-Rabin for 64-bit integers (bases 2..37). */
int orc_is_prime(uint64_t n) {
    static const u64 bases[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
    if (n < 2) return 0;
    for (int i = 0; i < 12; i++) { if (n == bases[i]) return 1; if (n % bases[i] == 0) return 0; }
    u64 d = n - 1; int s = 0; while (!(d & 1)) { d >>= 1; s++; }
    for (int i = 0; i < 12; i++) {
        u64 x = powmod(bases[i], d, n);
        if (x == 1 || x == n - 1) continue;
        int comp = 1;
        for (int r = 1; r < s; r++) { x = orc_mulmod(x, x, n); if (x == n - 1) { comp = 0; break; } }
        if (comp) return 0;
    }
    return 1;
}

/* Pollard-Brent rho, used to factor q-1 when searching a generator. */
static u64 gcd64(u64 a, u64 b) { while (b) { u64 t = a % b; a = b; b = t; } return a; }
static u64 rho(u64 n) {
    if (n % 2 == 0) return 2;
    for (u64 c = 1;; c++) {
        u64 y = 2, x = 2, g = 1, q = 1, ys = 2; u64 m = 128, r = 1;
        do {
            x = y;
            for (u64 i = 0; i < r; i++) y = (orc_mulmod(y, y, n) + c) % n;
            u64 k = 0;
            do {
                ys = y;
                for (u64 i = 0; i < m && i < r - k; i++) {
                    y = (orc_mulmod(y, y, n) + c) % n;
                    q = orc_mulmod(q, x > y ? x - y : y - x, n);
                }
                g = gcd64(q, n); k += m;
            } while (k < r && g == 1);
            r <<= 1;
        } while (g == 1);
        if (g == n) {
            do { ys = (orc_mulmod(ys, ys, n) + c) % n; g = gcd64(x > ys ? x - ys : ys - x, n); } while (g == 1);
        }
        if (g != n) return g;
    }
}
static int factor_rec(u64 n, u64* f, int nf) {
    if (n == 1) return nf;
    if (orc_is_prime(n)) { for (int i = 0; i < nf; i++) if (f[i] == n) return nf; f[nf] = n; return nf + 1; }
    for (u64 p = 2; p < 1000; p++) if (n % p == 0) { nf = factor_rec(p, f, nf); while (n % p == 0) n /= p; return factor_rec(n, f, nf); }
    u64 d = rho(n);
    nf = factor_rec(d, f, nf);
    return factor_rec(n / d, f, nf);
}
/* Smallest generator of Z_q^* (Lattigo ring.PrimitiveRoot searches upward from 2). */
static u64 smallest_generator(u64 q) {
    u64 f[64]; int nf = factor_rec(q - 1, f, 0);
    for (u64 g = 2;; g++) {
        int ok = 1;
        for (int i = 0; i < nf && ok; i++) if (powmod(g, (q - 1) / f[i], q) == 1) ok = 0;
        if (ok) return g;
    }
}

/* NTT-friendly prime chain, restating Lattigo's rlwe.GenModuli: primes are
 * grouped by bit size; each size draws from a generator of candidates
 * 2^b + 1 +/- k*2N; 61-bit sizes go downstream only, other sizes alternate
 * upstream/downstream starting upstream; Q takes its primes first, then P.
 * (scheme.go:58-66 reaches this through ckks.NewParametersFromLiteral.) */
typedef struct { int bits; u64 up, down; int next_up; } pgen_t;
static u64 pgen_next(pgen_t* g, u64 nth) {
    int up = g->bits == 61 ? 0 : g->next_up;
    if (g->bits != 61) g->next_up = !g->next_up;
    for (;;) {
        u64 cand;
        if (up) { g->up += nth; cand = g->up; } else { g->down -= nth; cand = g->down; }
        if (orc_is_prime(cand)) return cand;
    }
}
int orc_gen_primes(int logN, const int* logq, int nq, const int* logp, int np,
                   uint64_t* q_out, uint64_t* p_out) {
    u64 nth = (u64)2 << logN;
    pgen_t gens[64]; int ng = 0;
    u64* outs[2] = {q_out, p_out}; const int* bits[2] = {logq, logp}; int cnt[2] = {nq, np};
    for (int s = 0; s < 2; s++) for (int i = 0; i < cnt[s]; i++) {
        int b = bits[s][i];
        if (b < 10 || b > 61) return -1;
        int gi = -1;
        for (int k = 0; k < ng; k++) if (gens[k].bits == b) gi = k;
        if (gi < 0) { gi = ng++; gens[gi].bits = b; gens[gi].up = ((u64)1 << b) + 1; gens[gi].down = ((u64)1 << b) + 1; gens[gi].next_up = 1; }
        outs[s][i] = pgen_next(&gens[gi], nth);
    }
    return 0;
}

/* =====================================================================
 * 2. Counter PRNG and samplers (own construction; Lattigo's keyed PRNG is
 *    not reproducible without the Go module -- keys and encryption
 *    randomness are inputs to parity, generated identically by the
 *    product from the same seed).
 *    rand64(seed, stream, ctr) = mix(mix(seed + G*(stream+1)) ^ (ctr*M1 + M2))
 *    with mix the splitmix64 finaliser (Steele, Lea, Flood 2014).
 * ===================================================================== */
static inline u64 mix64(u64 z) {
    z ^= z >> 30; z *= 0xbf58476d1ce4e5b9ULL;
    z ^= z >> 27; z *= 0x94d049bb133111ebULL;
    z ^= z >> 31; return z;
}
uint64_t orc_rand64(uint64_t seed, uint64_t stream, uint64_t ctr) {
    u64 k = mix64(seed + 0x9e3779b97f4a7c15ULL * (stream + 1));
    return mix64(k ^ (ctr * 0xd1b54a32d192ed03ULL + 0x8cb92ba72f3d8dd7ULL));
}
#define ST_SK 1ULL
#define ST_PK_A 2ULL
#define ST_PK_E 3ULL
#define ST_GK_A(g, d) ((4ULL << 56) | ((u64)(g) << 8) | (u64)(d))
#define ST_GK_E(g, d) ((5ULL << 56) | ((u64)(g) << 8) | (u64)(d))
#define ST_ENC_U(e) ((6ULL << 56) | (u64)(e))
#define ST_ENC_E0(e) ((7ULL << 56) | (u64)(e))
#define ST_ENC_E1(e) ((8ULL << 56) | (u64)(e))
#define ST_RLK_A(d) ((9ULL << 56) | (u64)(d))
#define ST_RLK_E(d) ((10ULL << 56) | (u64)(d))
#define ST_SEED_A (11ULL << 56)
#define ST_SEED_E(e) ((12ULL << 56) | (u64)(e))

static inline u64 uniform_mod(u64 r, u64 q) { return (u64)(((u128)r * q) >> 64); }
/* centred binomial, eta = 21 per side: sigma = sqrt(21/2) ~ 3.24 */
static inline i64 cbd21(u64 r) {
    return (i64)__builtin_popcountll(r & 0x1FFFFFULL) - (i64)__builtin_popcountll((r >> 21) & 0x1FFFFFULL);
}
/* ternary with exactly h nonzero +-1 coefficients (partial Fisher-Yates) */
static void sample_ternary_hw(u64 seed, u64 stream, int N, int h, i64* out) {
    int* idx = (int*)xmalloc(sizeof(int) * N);
    for (int i = 0; i < N; i++) { idx[i] = i; out[i] = 0; }
    if (h > N) h = N;
    for (int k = 0; k < h; k++) {
        u64 r = orc_rand64(seed, stream, (u64)k);
        int j = k + (int)(((u128)r * (u64)(N - k)) >> 64);
        int t = idx[k]; idx[k] = idx[j]; idx[j] = t;
        out[idx[k]] = (orc_rand64(seed, stream, (1ULL << 32) + (u64)k) & 1) ? -1 : 1;
    }
    free(idx);
}
static inline u64 signed_mod(i64 v, u64 q) { return v >= 0 ? (u64)v % q : negmod((u64)(-v) % q, q); }

/* =====================================================================
 * 3. Context, NTT tables
 * ===================================================================== */
struct gk_entry { u64 galel; u64* key; };
struct orc_ctx {
    int logN, N, L, K, h, dnum;
    u64 seed;
    u64 mod[MAXMOD];
    barrett_t bar[MAXMOD];
    u64 *psi, *psip, *ipsi, *ipsip; /* [mod][N] Shoup tables, bit-reversed */
    u64 ninv[MAXMOD], ninvp[MAXMOD];
    i64* s;          /* ternary secret (coefficients) */
    u64* s_ntt;      /* [L+K][N] */
    u64* pk;         /* [2][L+K][N] */
    struct gk_entry* gk; int ngk, capgk;
    u64* rlk;        /* relinearization key [dnum][2][L+K][N], or NULL */
    /* encoder */
    double *rre, *rim; /* roots of unity exp(2 pi i k / M), k = 0..M */
    int* rotgroup;   /* 5^j mod M */
};

static inline u64 M_(const orc_ctx* c, int i) { return c->mod[i]; }
int orc_N(const orc_ctx* c) { return c->N; }
uint64_t orc_modulus(const orc_ctx* c, int idx) { return c->mod[idx]; }
static inline int brv(int x, int logn) { int r = 0; for (int i = 0; i < logn; i++) { r = (r << 1) | (x & 1); x >>= 1; } return r; }

static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

static void init_ntt_tables(orc_ctx* c) {
    int N = c->N, nm = c->L + c->K;
    c->psi = (u64*)xmalloc(8 * (size_t)nm * N); c->psip = (u64*)xmalloc(8 * (size_t)nm * N);
    c->ipsi = (u64*)xmalloc(8 * (size_t)nm * N); c->ipsip = (u64*)xmalloc(8 * (size_t)nm * N);
    for (int m = 0; m < nm; m++) {
        u64 q = c->mod[m];
        if ((q - 1) % (2 * (u64)N)) die("modulus is not 1 mod 2N");
        u64 g = smallest_generator(q);
        u64 psi = powmod(g, (q - 1) / (2 * (u64)N), q), ipsi = invmod_prime(psi, q);
        u64* pw = (u64*)xmalloc(8 * (size_t)N); u64* ipw = (u64*)xmalloc(8 * (size_t)N);
        pw[0] = 1; ipw[0] = 1;
        for (int i = 1; i < N; i++) { pw[i] = orc_mulmod(pw[i - 1], psi, q); ipw[i] = orc_mulmod(ipw[i - 1], ipsi, q); }
        for (int i = 0; i < N; i++) {
            int r = brv(i, c->logN);
            c->psi[(size_t)m * N + i] = pw[r]; c->psip[(size_t)m * N + i] = shoup_pre(pw[r], q);
            c->ipsi[(size_t)m * N + i] = ipw[r]; c->ipsip[(size_t)m * N + i] = shoup_pre(ipw[r], q);
        }
        c->ninv[m] = invmod_prime((u64)N, q); c->ninvp[m] = shoup_pre(c->ninv[m], q);
        free(pw); free(ipw);
    }
}

/* Forward negacyclic NTT, Cooley-Tukey with bit-reversed psi powers
 * (Longa-Naehrig 2016, Alg. 1): natural-order input, output slot j holds
 * a(psi^(2 brv(j) + 1)) -- Lattigo's NTT ordering. */
void orc_ntt(const orc_ctx* c, int m, uint64_t* a) {
    int N = c->N; u64 q = c->mod[m];
    const u64* W = c->psi + (size_t)m * N; const u64* Wp = c->psip + (size_t)m * N;
    int t = N;
    for (int mm = 1; mm < N; mm <<= 1) {
        t >>= 1;
        for (int i = 0; i < mm; i++) {
            int j1 = 2 * i * t; u64 w = W[mm + i], wp = Wp[mm + i];
            for (int j = j1; j < j1 + t; j++) {
                u64 U = a[j], V = shoup_mul(a[j + t], w, wp, q);
                a[j] = addmod(U, V, q); a[j + t] = submod(U, V, q);
            }
        }
    }
}
/* Inverse negacyclic NTT, Gentleman-Sande (Longa-Naehrig 2016, Alg. 2). */
void orc_intt(const orc_ctx* c, int m, uint64_t* a) {
    int N = c->N; u64 q = c->mod[m];
    const u64* W = c->ipsi + (size_t)m * N; const u64* Wp = c->ipsip + (size_t)m * N;
    int t = 1;
    for (int mm = N; mm > 1; mm >>= 1) {
        int h = mm >> 1, j1 = 0;
        for (int i = 0; i < h; i++) {
            u64 w = W[h + i], wp = Wp[h + i];
            for (int j = j1; j < j1 + t; j++) {
                u64 U = a[j], V = a[j + t];
                a[j] = addmod(U, V, q); a[j + t] = shoup_mul(submod(U, V, q), w, wp, q);
            }
            j1 += 2 * t;
        }
        t <<= 1;
    }
    for (int j = 0; j < N; j++) a[j] = shoup_mul(a[j], c->ninv[m], c->ninvp[m], q);
}

/* limb helpers over a list of modulus indices */
static void ntt_limbs(const orc_ctx* c, u64* a, const int* mi, int n) {
    #pragma omp parallel for num_threads(g_threads) schedule(static) if (n > 1 && g_threads > 1)
    for (int i = 0; i < n; i++) orc_ntt(c, mi[i], a + (size_t)i * c->N);
}
static void intt_limbs(const orc_ctx* c, u64* a, const int* mi, int n) {
    #pragma omp parallel for num_threads(g_threads) schedule(static) if (n > 1 && g_threads > 1)
    for (int i = 0; i < n; i++) orc_intt(c, mi[i], a + (size_t)i * c->N);
}
/* modulus-index list of a Q poly at level l, and of a QP poly at level l */
static int q_list(const orc_ctx* c, int l, int* mi) { (void)c; for (int i = 0; i <= l; i++) mi[i] = i; return l + 1; }
static int qp_list(const orc_ctx* c, int l, int* mi) {
    int n = 0; for (int i = 0; i <= l; i++) mi[n++] = i;
    for (int j = 0; j < c->K; j++) mi[n++] = c->L + j;
    return n;
}

uint64_t orc_galois_element(const orc_ctx* c, int k) {
    /* Lattigo Parameters.GaloisElement: 5^k mod 2N, k taken mod 2N (two's complement) */
    u64 M = (u64)2 * c->N; u64 e = (u64)((i64)k) & (M - 1);
    return powmod(5, e, M);
}
/* Lattigo ring.AutomorphismNTTIndex: out[i] = in[idx[i]] */
void orc_automorphism_index(const orc_ctx* c, uint64_t galel, uint32_t* idx) {
    int N = c->N, logN = c->logN; u64 mask = 2 * (u64)N - 1;
    for (int i = 0; i < N; i++) {
        u64 e = 2 * (u64)brv(i, logN) + 1;
        u64 t = ((galel * e) & mask) - 1;
        idx[i] = (uint32_t)brv((int)(t >> 1), logN);
    }
}
static void permute_limbs(const orc_ctx* c, const u64* in, u64* out, int nl, const uint32_t* idx) {
    int N = c->N;
    for (int l = 0; l < nl; l++) for (int i = 0; i < N; i++) out[(size_t)l * N + i] = in[(size_t)l * N + idx[i]];
}

/* =====================================================================
 * 4. Basis extension (Lattigo ring.ModUpExact / Decomposer.DecomposeAndSplit):
 *    y_i = x_i * [(S/s_i)^-1]_{s_i};  v = (u64) sum_i (double)y_i/(double)s_i
 *    (float64, left to right, truncated);  out_t = sum_i y_i*[S/s_i]_t - v*[S]_t.
 * ===================================================================== */
typedef struct { int ns, nd; u64 hatinv[MAXMOD]; u64* hat; /* [nd][ns] */ u64 Smod[MAXMOD]; } bconv_t;
static void bconv_make(const orc_ctx* c, const int* src, int ns, const int* dst, int nd, bconv_t* b) {
    b->ns = ns; b->nd = nd; b->hat = (u64*)xmalloc(8 * (size_t)ns * nd);
    for (int i = 0; i < ns; i++) {
        u64 si = M_(c, src[i]); u64 pr = 1;
        for (int j = 0; j < ns; j++) if (j != i) pr = orc_mulmod(pr, M_(c, src[j]) % si, si);
        b->hatinv[i] = invmod_prime(pr, si);
    }
    for (int k = 0; k < nd; k++) {
        u64 t = M_(c, dst[k]); u64 S = 1;
        for (int j = 0; j < ns; j++) S = orc_mulmod(S, M_(c, src[j]) % t, t);
        b->Smod[k] = S;
        for (int i = 0; i < ns; i++) {
            u64 pr = 1;
            for (int j = 0; j < ns; j++) if (j != i) pr = orc_mulmod(pr, M_(c, src[j]) % t, t);
            b->hat[(size_t)k * ns + i] = pr;
        }
    }
}
static void bconv_run(const orc_ctx* c, const int* src, const int* dst, const bconv_t* b, const u64* in, u64* out) {
    int N = c->N, ns = b->ns, nd = b->nd;
    #pragma omp parallel for num_threads(g_threads) schedule(static) if (g_threads > 1)
    for (int x = 0; x < N; x++) {
        u64 y[MAXMOD]; double vf = 0.0;
        for (int i = 0; i < ns; i++) {
            u64 si = M_(c, src[i]);
            y[i] = mulmod_b(&c->bar[src[i]], in[(size_t)i * N + x] % si, b->hatinv[i]);
            vf += (double)y[i] / (double)si;
        }
        u64 v = (u64)vf;
        for (int k = 0; k < nd; k++) {
            u64 t = M_(c, dst[k]); const u64* h = b->hat + (size_t)k * ns;
            u128 acc = 0; u64 r = 0;
            for (int i = 0; i < ns; i++) {
                acc += (u128)y[i] * h[i];
                if ((i & 7) == 7) { r = addmod(r, (u64)(acc % t), t); acc = 0; }
            }
            r = addmod(r, (u64)(acc % t), t);
            u64 vs = orc_mulmod(v % t, b->Smod[k], t);
            out[(size_t)k * N + x] = submod(r, vs, t);
        }
    }
}
void orc_basis_extend(const orc_ctx* c, const int* src, int ns, const int* dst, int nd,
                      const uint64_t* in, uint64_t* out) {
    bconv_t b; bconv_make(c, src, ns, dst, nd, &b); bconv_run(c, src, dst, &b, in, out); free(b.hat);
}

/* Decomposition of c1 (NTT domain, level l) into ceil((l+1)/K) RNS digits,
 * each extended to QP (Lattigo Evaluator.DecomposeNTT/DecomposeSingleNTT):
 * digits[d] is a QP poly at level l ((l+1+K) limbs, NTT domain).  The digit's
 * own limbs are copied from c1; a one-limb digit is reduced mod every other
 * modulus instead of extended. */
void orc_decompose_modup(const orc_ctx* c, int l, const uint64_t* c1, uint64_t* digits) {
    int N = c->N, K = c->K, nqp = l + 1 + K;
    int dn = (l + 1 + K - 1) / K;
    int qpl[MAXMOD]; qp_list(c, l, qpl);
    int ql[MAXMOD]; q_list(c, l, ql);
    u64* coef = (u64*)xmalloc(8 * (size_t)(l + 1) * N);
    memcpy(coef, c1, 8 * (size_t)(l + 1) * N);
    intt_limbs(c, coef, ql, l + 1);
    for (int d = 0; d < dn; d++) {
        u64* D = digits + (size_t)d * nqp * N;
        int st = d * K, en = st + K; if (en > l + 1) en = l + 1;
        int ns = en - st;
        int src[MAXMOD], dst[MAXMOD], dpos[MAXMOD], nd = 0;
        for (int i = 0; i < ns; i++) src[i] = st + i;
        for (int k = 0; k < nqp; k++) if (!(k >= st && k < en)) { dst[nd] = qpl[k]; dpos[nd] = k; nd++; }
        u64* tmp = (u64*)xmalloc(8 * (size_t)nd * N);
        if (ns == 1) {
            for (int k = 0; k < nd; k++) { u64 t = M_(c, dst[k]); for (int x = 0; x < N; x++) tmp[(size_t)k * N + x] = coef[(size_t)st * N + x] % t; }
        } else {
            orc_basis_extend(c, src, ns, dst, nd, coef + (size_t)st * N, tmp);
        }
        ntt_limbs(c, tmp, dst, nd);
        for (int k = 0; k < nd; k++) memcpy(D + (size_t)dpos[k] * N, tmp + (size_t)k * N, 8 * (size_t)N);
        for (int i = st; i < en; i++) memcpy(D + (size_t)i * N, c1 + (size_t)i * N, 8 * (size_t)N);
        free(tmp);
    }
    free(coef);
}

/* ModDown QP -> Q (Lattigo BasisExtender.ModDownQPtoQNTT): iNTT the P part,
 * extend [x]_P to Q exactly (float-v method over all K P limbs), NTT, and
 * return (x_Q - ext) * P^-1 mod q_i. */
void orc_mod_down(const orc_ctx* c, int l, const uint64_t* qp, uint64_t* q_out) {
    int N = c->N, K = c->K;
    int pl[MAXMOD], ql[MAXMOD];
    for (int j = 0; j < K; j++) pl[j] = c->L + j;
    q_list(c, l, ql);
    u64* pc = (u64*)xmalloc(8 * (size_t)K * N);
    memcpy(pc, qp + (size_t)(l + 1) * N, 8 * (size_t)K * N);
    intt_limbs(c, pc, pl, K);
    u64* ext = (u64*)xmalloc(8 * (size_t)(l + 1) * N);
    orc_basis_extend(c, pl, K, ql, l + 1, pc, ext);
    ntt_limbs(c, ext, ql, l + 1);
    for (int i = 0; i <= l; i++) {
        u64 q = c->mod[i]; u64 P = 1;
        for (int j = 0; j < K; j++) P = orc_mulmod(P, c->mod[c->L + j] % q, q);
        u64 Pinv = invmod_prime(P, q);
        for (int x = 0; x < N; x++)
            q_out[(size_t)i * N + x] = mulmod_b(&c->bar[i], submod(qp[(size_t)i * N + x], ext[(size_t)i * N + x], q), Pinv);
    }
    free(pc); free(ext);
}
/* Coefficient-domain ModDown from Q + {p_0} (Lattigo ModDownQPtoQ at levelP = 0,
 * used by public-key encryption). in: [(l+1)+1][N] coefficient domain. */
static void mod_down_p0_coeff(const orc_ctx* c, int l, const u64* in, u64* out) {
    int N = c->N; int src[1] = {c->L}; int ql[MAXMOD] = {0}; q_list(c, l, ql);
    u64* ext = (u64*)xmalloc(8 * (size_t)(l + 1) * N);
    orc_basis_extend(c, src, 1, ql, l + 1, in + (size_t)(l + 1) * N, ext);
    u64 p0 = c->mod[c->L];
    for (int i = 0; i <= l; i++) {
        u64 q = c->mod[i]; u64 Pinv = invmod_prime(p0 % q, q);
        for (int x = 0; x < N; x++)
            out[(size_t)i * N + x] = mulmod_b(&c->bar[i], submod(in[(size_t)i * N + x], ext[(size_t)i * N + x], q), Pinv);
    }
    free(ext);
}

/* =====================================================================
 * 5. Encoder (Lattigo ckks.Encoder, Standard ring, LogSlots = LogN-1)
 * ===================================================================== */
static void init_encoder(orc_ctx* c) {
    int M = 2 * c->N, slots = c->N / 2, quarm = M >> 2;
    c->rre = (double*)xcalloc(sizeof(double) * (M + 1)); c->rim = (double*)xcalloc(sizeof(double) * (M + 1));
    double angle = 2.0 * 3.141592653589793 / (double)M;
    /* Lattigo's root table: cosines of the first quadrant, the rest by symmetry */
    for (int i = 0; i < quarm; i++) { c->rre[i] = cos(angle * (double)i); c->rim[i] = 0.0; }
    for (int i = 0; i < quarm; i++) c->rim[quarm - i] += c->rre[i];
    for (int i = 1; i < quarm + 1; i++) { c->rre[i + quarm] = -c->rre[quarm - i]; c->rim[i + quarm] = c->rim[quarm - i]; }
    for (int i = 1; i < quarm + 1; i++) { c->rre[i + 2 * quarm] = -c->rre[i]; c->rim[i + 2 * quarm] = -c->rim[i]; }
    for (int i = 1; i < quarm; i++) { c->rre[i + 3 * quarm] = c->rre[quarm - i]; c->rim[i + 3 * quarm] = -c->rim[quarm - i]; }
    c->rre[M] = c->rre[0]; c->rim[M] = c->rim[0];
    c->rotgroup = (int*)xmalloc(sizeof(int) * slots);
    u64 p = 1;
    for (int j = 0; j < slots; j++) { c->rotgroup[j] = (int)p; p = (p * 5) & (u64)(M - 1); }
}
static void bitrev_cplx(double* re, double* im, int n) {
    int logn = 0; while ((1 << logn) < n) logn++;
    for (int i = 0; i < n; i++) { int j = brv(i, logn); if (j > i) { double t = re[i]; re[i] = re[j]; re[j] = t; t = im[i]; im[i] = im[j]; im[j] = t; } }
}
/* SpecialIFFT (HEAAN/Lattigo): butterflies with inverse rotation-group roots, then bit reversal, then /n */
static void special_ifft(const orc_ctx* c, double* re, double* im, int n) {
    int M = 2 * c->N;
    for (int len = n; len >= 2; len >>= 1) {
        int lenh = len >> 1, lenq = len << 2, gap = M / lenq, mask = lenq - 1;
        for (int i = 0; i < n; i += len) for (int j = 0; j < lenh; j++) {
            int k = i + j;
            double ur = re[k], ui = im[k], vr = re[k + lenh], vi = im[k + lenh];
            int idx = (lenq - (c->rotgroup[j] & mask)) * gap;
            double wr = c->rre[idx], wi = c->rim[idx];
            double dr = ur - vr, di = ui - vi;
            re[k] = ur + vr; im[k] = ui + vi;
            re[k + lenh] = dr * wr - di * wi; im[k + lenh] = dr * wi + di * wr;
        }
    }
    bitrev_cplx(re, im, n);
    for (int i = 0; i < n; i++) { re[i] /= (double)n; im[i] /= (double)n; }
}
/* SpecialFFT (HEAAN/Lattigo): bit reversal, then butterflies with rotation-group roots */
static void special_fft(const orc_ctx* c, double* re, double* im, int n) {
    int M = 2 * c->N;
    bitrev_cplx(re, im, n);
    for (int len = 2; len <= n; len <<= 1) {
        int lenh = len >> 1, lenq = len << 2, gap = M / lenq, mask = lenq - 1;
        for (int i = 0; i < n; i += len) for (int j = 0; j < lenh; j++) {
            int k = i + j;
            int idx = (c->rotgroup[j] & mask) * gap;
            double wr = c->rre[idx], wi = c->rim[idx];
            double ur = re[k], ui = im[k];
            double xr = re[k + lenh], xi = im[k + lenh];
            double vr = xr * wr - xi * wi, vi = xr * wi + xi * wr;
            re[k] = ur + vr; im[k] = ui + vi;
            re[k + lenh] = ur - vr; im[k + lenh] = ui - vi;
        }
    }
}
/* Lattigo SingleFloat64ToFixedPointCRT: |v|*scale, +0.5 and truncate below
 * 2^64 (float64 arithmetic), exact big-integer path above; negate mod q. */
static void fixed_point_crt(const orc_ctx* c, double value, double scale, const int* mi, int nm, u64* out, size_t stride) {
    if (value == 0) { for (int j = 0; j < nm; j++) out[(size_t)j * stride] = 0; return; }
    int neg = 0;
    if (value < 0) { neg = 1; scale *= -1; }
    value *= scale;
    if (value >= 1.8446744073709552e+19) {
        int e; double m = frexp(value, &e); /* value = m * 2^e, m in [0.5,1) */
        u64 mant = (u64)ldexp(m, 53); int sh = e - 53;
        for (int j = 0; j < nm; j++) {
            u64 q = c->mod[mi[j]];
            u64 r = orc_mulmod(mant % q, powmod(2, (u64)sh, q), q);
            out[(size_t)j * stride] = neg ? negmod(r, q) : r;
        }
    } else {
        u64 cc = (u64)(value + 0.5);
        for (int j = 0; j < nm; j++) {
            u64 q = c->mod[mi[j]]; u64 r = cc % q;
            out[(size_t)j * stride] = neg ? negmod(r, q) : r;
        }
    }
}
/* Complex slots (Lattigo Encoder.Encode of []complex128, encoder.go:50-70):
 * vi may be NULL (real input). */
void orc_encode_complex_f64(const orc_ctx* c, const double* v, const double* vi, int n, int level, double scale, int with_p,
                            uint64_t* out) {
    int N = c->N, slots = N / 2;
    double* re = (double*)xcalloc(sizeof(double) * slots); double* im = (double*)xcalloc(sizeof(double) * slots);
    for (int i = 0; i < n && i < slots; i++) { re[i] = v[i]; if (vi) im[i] = vi[i]; }
    special_ifft(c, re, im, slots);
    int mi[MAXMOD]; int nm = with_p ? qp_list(c, level, mi) : q_list(c, level, mi);
    for (int i = 0; i < slots; i++) {
        fixed_point_crt(c, re[i], scale, mi, nm, out + i, (size_t)N);
        fixed_point_crt(c, im[i], scale, mi, nm, out + i + slots, (size_t)N);
    }
    ntt_limbs(c, out, mi, nm);
    free(re); free(im);
}
void orc_encode_f64(const orc_ctx* c, const double* v, int n, int level, double scale, int with_p, uint64_t* out) {
    orc_encode_complex_f64(c, v, NULL, n, level, scale, with_p, out);
}
/* EncodeComplex's fp32 interleaved input [re0, im0, re1, im1, ...] of n values */
void orc_encode_complex(const orc_ctx* c, const float* v, int n, int level, double scale, uint64_t* out) {
    double* re = (double*)xmalloc(sizeof(double) * (n > 0 ? n : 1));
    double* im = (double*)xmalloc(sizeof(double) * (n > 0 ? n : 1));
    for (int i = 0; i < n; i++) { re[i] = (double)v[2 * i]; im[i] = (double)v[2 * i + 1]; }
    orc_encode_complex_f64(c, re, im, n, level, scale, 0, out);
    free(re); free(im);
}
void orc_encode(const orc_ctx* c, const float* v, int n, int level, double scale, int with_p, uint64_t* out) {
    double* d = (double*)xmalloc(sizeof(double) * (n > 0 ? n : 1));
    for (int i = 0; i < n; i++) d[i] = (double)v[i];
    orc_encode_f64(c, d, n, level, scale, with_p, out);
    free(d);
}

/* ---- big integers (little-endian u64 words) for CRT decoding ---- */
typedef struct { int n; u64 w[BIGW]; } big_t;
static void big_from_u64(big_t* a, u64 x) { memset(a, 0, sizeof(*a)); a->w[0] = x; a->n = x ? 1 : 0; }
static void big_norm(big_t* a) { while (a->n > 0 && a->w[a->n - 1] == 0) a->n--; }
static void big_mul_u64(big_t* a, u64 m) {
    u128 carry = 0;
    for (int i = 0; i < a->n; i++) { u128 t = (u128)a->w[i] * m + carry; a->w[i] = (u64)t; carry = t >> 64; }
    if (carry) { a->w[a->n] = (u64)carry; a->n++; }
    big_norm(a);
}
static int big_cmp(const big_t* a, const big_t* b) {
    if (a->n != b->n) return a->n < b->n ? -1 : 1;
    for (int i = a->n - 1; i >= 0; i--) if (a->w[i] != b->w[i]) return a->w[i] < b->w[i] ? -1 : 1;
    return 0;
}
static void big_add(big_t* a, const big_t* b) {
    int n = a->n > b->n ? a->n : b->n; u64 carry = 0;
    for (int i = 0; i < n; i++) {
        u64 x = i < a->n ? a->w[i] : 0, y = i < b->n ? b->w[i] : 0;
        u128 t = (u128)x + y + carry; a->w[i] = (u64)t; carry = (u64)(t >> 64);
    }
    a->n = n; if (carry) { a->w[n] = carry; a->n++; }
}
static void big_sub(big_t* a, const big_t* b) { /* a >= b */
    u64 borrow = 0;
    for (int i = 0; i < a->n; i++) {
        u64 y = i < b->n ? b->w[i] : 0;
        u128 t = (u128)a->w[i] - y - borrow; a->w[i] = (u64)t; borrow = (u64)(t >> 64) ? 1 : 0;
    }
    big_norm(a);
}
static void big_shr1(big_t* a) {
    for (int i = 0; i < a->n; i++) a->w[i] = (a->w[i] >> 1) | (i + 1 < a->n ? a->w[i + 1] << 63 : 0);
    big_norm(a);
}
/* nearest double (round half to even), as big.Float.Float64 */
static double big_to_double(const big_t* a) {
    if (a->n == 0) return 0.0;
    int top = a->n - 1; int lz = __builtin_clzll(a->w[top]);
    int bitlen = top * 64 + (64 - lz);
    if (bitlen <= 64) return (double)a->w[0];
    int sh = bitlen - 64; /* extract bits [sh, sh+64) */
    int wi = sh / 64, bi = sh % 64;
    u64 hi = bi ? (a->w[wi] >> bi) | (a->w[wi + 1] << (64 - bi)) : a->w[wi];
    int sticky = 0;
    if (bi && (a->w[wi] & ((1ULL << bi) - 1))) sticky = 1;
    for (int i = 0; i < wi; i++) if (a->w[i]) sticky = 1;
    if (sticky) hi |= 1;
    return ldexp((double)hi, sh);
}

/* Lattigo Encoder.Decode (float64 path): iNTT, centred CRT reconstruction to
 * a big integer, nearest double, divide by the scale, SpecialFFT. */
static void decode_core(const orc_ctx* c, const uint64_t* pt, int level, double scale, double* out, double* out_im);
void orc_decode_f64(const orc_ctx* c, const uint64_t* pt, int level, double scale, double* out) {
    decode_core(c, pt, level, scale, out, NULL);
}
/* DecodeComplex (encoder.go:72-91): interleaved [re0, im0, re1, im1, ...] */
void orc_decode_complex_f64(const orc_ctx* c, const uint64_t* pt, int level, double scale, double* out) {
    int slots = c->N / 2;
    double* re = (double*)xmalloc(sizeof(double) * slots); double* im = (double*)xmalloc(sizeof(double) * slots);
    decode_core(c, pt, level, scale, re, im);
    for (int i = 0; i < slots; i++) { out[2 * i] = re[i]; out[2 * i + 1] = im[i]; }
    free(re); free(im);
}
static void decode_core(const orc_ctx* c, const uint64_t* pt, int level, double scale, double* out, double* out_im) {
    int N = c->N, slots = N / 2, nl = level + 1;
    int ql[MAXMOD]; q_list(c, level, ql);
    u64* coef = (u64*)xmalloc(8 * (size_t)nl * N);
    memcpy(coef, pt, 8 * (size_t)nl * N);
    intt_limbs(c, coef, ql, nl);
    double* vals = (double*)xmalloc(sizeof(double) * N);
    if (level == 0) {
        u64 q = c->mod[0];
        for (int x = 0; x < N; x++) {
            u64 v = coef[x];
            vals[x] = v >= (q >> 1) ? -(double)(q - v) : (double)v;
            vals[x] /= scale;
        }
    } else {
        big_t Q; big_from_u64(&Q, 1);
        for (int i = 0; i < nl; i++) big_mul_u64(&Q, c->mod[i]);
        big_t Qh = Q; big_shr1(&Qh);
        big_t* hat = (big_t*)xmalloc(sizeof(big_t) * nl); u64 hinv[MAXMOD];
        for (int i = 0; i < nl; i++) {
            big_from_u64(&hat[i], 1); u64 pr = 1;
            for (int j = 0; j < nl; j++) if (j != i) { big_mul_u64(&hat[i], c->mod[j]); pr = orc_mulmod(pr, c->mod[j] % c->mod[i], c->mod[i]); }
            hinv[i] = invmod_prime(pr, c->mod[i]);
        }
        #pragma omp parallel for num_threads(g_threads) schedule(static) if (g_threads > 1)
        for (int x = 0; x < N; x++) {
            big_t acc; big_from_u64(&acc, 0);
            for (int i = 0; i < nl; i++) {
                u64 y = orc_mulmod(coef[(size_t)i * N + x], hinv[i], c->mod[i]);
                big_t t = hat[i]; big_mul_u64(&t, y); big_add(&acc, &t);
            }
            while (big_cmp(&acc, &Q) >= 0) big_sub(&acc, &Q);
            double d;
            if (big_cmp(&acc, &Qh) >= 0) { big_t t = Q; big_sub(&t, &acc); d = -big_to_double(&t); }
            else d = big_to_double(&acc);
            vals[x] = d / scale;
        }
        free(hat);
    }
    double* re = (double*)xmalloc(sizeof(double) * slots); double* im = (double*)xmalloc(sizeof(double) * slots);
    for (int i = 0; i < slots; i++) { re[i] = vals[i]; im[i] = vals[i + slots]; }
    special_fft(c, re, im, slots);
    for (int i = 0; i < slots; i++) out[i] = re[i];
    if (out_im) for (int i = 0; i < slots; i++) out_im[i] = im[i];
    free(re); free(im); free(vals); free(coef);
}
void orc_decode(const orc_ctx* c, const uint64_t* pt, int level, double scale, float* out) {
    int slots = c->N / 2; double* d = (double*)xmalloc(sizeof(double) * slots);
    orc_decode_f64(c, pt, level, scale, d);
    for (int i = 0; i < slots; i++) out[i] = (float)d[i];
    free(d);
}

/* =====================================================================
 * 6. Keys (Lattigo rlwe.KeyGenerator; keygenerator.go:13-35, evaluator.go:29-66)
 * ===================================================================== */
static void poly_from_signed(const orc_ctx* c, const i64* v, const int* mi, int nm, u64* out) {
    int N = c->N;
    #pragma omp parallel for num_threads(g_threads) schedule(static) if (nm > 1 && g_threads > 1)
    for (int j = 0; j < nm; j++) { u64 q = c->mod[mi[j]]; for (int x = 0; x < N; x++) out[(size_t)j * N + x] = signed_mod(v[x], q); }
}
static void sample_cbd(u64 seed, u64 stream, int N, i64* out) { for (int x = 0; x < N; x++) out[x] = cbd21(orc_rand64(seed, stream, (u64)x)); }
static void sample_uniform_qp(const orc_ctx* c, u64 stream, const int* mi, int nm, u64* out) {
    int N = c->N;
    #pragma omp parallel for num_threads(g_threads) schedule(static) if (nm > 1 && g_threads > 1)
    for (int j = 0; j < nm; j++) { u64 q = c->mod[mi[j]]; for (int x = 0; x < N; x++) out[(size_t)j * N + x] = uniform_mod(orc_rand64(c->seed, stream, (u64)mi[j] * N + x), q); }
}
static void full_qp_list(const orc_ctx* c, int* mi) { for (int i = 0; i < c->L + c->K; i++) mi[i] = i; }

static void init_keys(orc_ctx* c) {
    int N = c->N, nm = c->L + c->K; int mi[MAXMOD]; full_qp_list(c, mi);
    c->s = (i64*)xmalloc(sizeof(i64) * N);
    sample_ternary_hw(c->seed, ST_SK, N, c->h, c->s);
    c->s_ntt = (u64*)xmalloc(8 * (size_t)nm * N);
    poly_from_signed(c, c->s, mi, nm, c->s_ntt); ntt_limbs(c, c->s_ntt, mi, nm);
    /* public key (-a s + e, a) over the full QP basis */
    c->pk = (u64*)xmalloc(8 * (size_t)2 * nm * N);
    u64* b = c->pk; u64* a = c->pk + (size_t)nm * N;
    sample_uniform_qp(c, ST_PK_A, mi, nm, a); ntt_limbs(c, a, mi, nm);
    i64* e = (i64*)xmalloc(sizeof(i64) * N); sample_cbd(c->seed, ST_PK_E, N, e);
    poly_from_signed(c, e, mi, nm, b); ntt_limbs(c, b, mi, nm);
    for (int j = 0; j < nm; j++) { u64 q = c->mod[j]; for (int x = 0; x < N; x++) { size_t o = (size_t)j * N + x; b[o] = submod(b[o], mulmod_b(&c->bar[j], a[o], c->s_ntt[o]), q); } }
    free(e);
}
void orc_secret_key(const orc_ctx* c, int64_t* s) { memcpy(s, c->s, sizeof(i64) * c->N); }
void orc_public_key(const orc_ctx* c, uint64_t* out) { memcpy(out, c->pk, 8 * (size_t)2 * (c->L + c->K) * c->N); }

/* Galois key for galel: dnum digits of (b_d, a_d) over QP, b_d = -a_d*s' + e_d
 * + [P*s on the limbs of digit d], s' = sigma_{galel^-1}(s)
 * (Lattigo KeyGenerator.GenGaloisKey: encrypts s under pi_{k^-1}(s)). */
/* Evaluation key from s_in to s_out (both NTT over QP): dnum digits of
 * (b_d, a_d), b_d = -a_d*s_out + e_d + [P*s_in on the limbs of digit d]
 * (Lattigo KeyGenerator.GenEvaluationKey).  a_d is sampled uniformly in the
 * NTT domain, as Lattigo samples it (a uniform polynomial is uniform in
 * either domain), word (m, x) = uniform_mod(rand64(seed, stream, m*N + x)). */
static u64* gen_eval_key(orc_ctx* c, const u64* s_in_ntt, const u64* s_out_ntt, u64 (*st_a)(u64, u64),
                         u64 (*st_e)(u64, u64), u64 tag) {
    int N = c->N, nm = c->L + c->K, K = c->K; int mi[MAXMOD]; full_qp_list(c, mi);
    u64* key = (u64*)xmalloc(8 * (size_t)c->dnum * 2 * nm * N);
    i64* e = (i64*)xmalloc(sizeof(i64) * N);
    for (int d = 0; d < c->dnum; d++) {
        u64* b = key + (size_t)d * 2 * nm * N; u64* a = b + (size_t)nm * N;
        sample_uniform_qp(c, st_a(tag, (u64)d), mi, nm, a);
        sample_cbd(c->seed, st_e(tag, (u64)d), N, e);
        poly_from_signed(c, e, mi, nm, b); ntt_limbs(c, b, mi, nm);
        #pragma omp parallel for num_threads(g_threads) schedule(static) if (g_threads > 1)
        for (int j = 0; j < nm; j++) {
            u64 q = c->mod[j]; u64 Pq = 0; int own = (j < c->L) && (j >= d * K) && (j < (d + 1) * K);
            if (own) { Pq = 1; for (int k = 0; k < K; k++) Pq = orc_mulmod(Pq, c->mod[c->L + k] % q, q); }
            for (int x = 0; x < N; x++) {
                size_t o = (size_t)j * N + x;
                u64 v = submod(b[o], mulmod_b(&c->bar[j], a[o], s_out_ntt[o]), q);
                if (own) v = addmod(v, mulmod_b(&c->bar[j], Pq, s_in_ntt[o]), q);
                b[o] = v;
            }
        }
    }
    free(e);
    return key;
}
static u64 st_gk_a(u64 g, u64 d) { return ST_GK_A(g, d); }
static u64 st_gk_e(u64 g, u64 d) { return ST_GK_E(g, d); }
static u64 st_rlk_a(u64 g, u64 d) { (void)g; return ST_RLK_A(d); }
static u64 st_rlk_e(u64 g, u64 d) { (void)g; return ST_RLK_E(d); }
static u64* gen_galois_key(orc_ctx* c, u64 galel) {
    int N = c->N, nm = c->L + c->K; int mi[MAXMOD]; full_qp_list(c, mi);
    u64 M = 2 * (u64)N; u64 ginv = invmod_generic(galel, M);
    i64* so = (i64*)xcalloc(sizeof(i64) * N);
    for (int i = 0; i < N; i++) { u64 t = ((u64)i * ginv) % M; if (t < (u64)N) so[t] += c->s[i]; else so[t - N] -= c->s[i]; }
    u64* so_ntt = (u64*)xmalloc(8 * (size_t)nm * N);
    poly_from_signed(c, so, mi, nm, so_ntt); ntt_limbs(c, so_ntt, mi, nm);
    u64* key = gen_eval_key(c, c->s_ntt, so_ntt, st_gk_a, st_gk_e, galel);
    free(so); free(so_ntt);
    return key;
}
/* Relinearization key: s^2 -> s (Lattigo KeyGenerator.GenRelinearizationKey). */
const uint64_t* orc_relin_key(orc_ctx* c) {
    if (c->rlk) return c->rlk;
    int N = c->N, nm = c->L + c->K;
    u64* s2 = (u64*)xmalloc(8 * (size_t)nm * N);
    for (int j = 0; j < nm; j++) for (int x = 0; x < N; x++) {
        size_t o = (size_t)j * N + x; s2[o] = mulmod_b(&c->bar[j], c->s_ntt[o], c->s_ntt[o]);
    }
    c->rlk = gen_eval_key(c, s2, c->s_ntt, st_rlk_a, st_rlk_e, 0);
    free(s2);
    return c->rlk;
}
const uint64_t* orc_galois_key(orc_ctx* c, uint64_t galel) {
    for (int i = 0; i < c->ngk; i++) if (c->gk[i].galel == galel) return c->gk[i].key;
    if (c->ngk == c->capgk) { c->capgk = c->capgk ? 2 * c->capgk : 16; c->gk = (struct gk_entry*)realloc(c->gk, sizeof(struct gk_entry) * c->capgk); }
    c->gk[c->ngk].galel = galel; c->gk[c->ngk].key = gen_galois_key(c, galel);
    return c->gk[c->ngk++].key;
}

/* ===================================================================== */
orc_ctx* orc_new(int logN, const uint64_t* q, int L, const uint64_t* p, int K, int h, uint64_t seed) {
    if (L + K > MAXMOD || K < 1 || L < 1 || logN < 2 || logN > 17) return NULL;
    orc_ctx* c = (orc_ctx*)xcalloc(sizeof(orc_ctx));
    c->logN = logN; c->N = 1 << logN; c->L = L; c->K = K; c->h = h; c->seed = seed;
    c->dnum = (L + K - 1) / K;
    for (int i = 0; i < L; i++) c->mod[i] = q[i];
    for (int j = 0; j < K; j++) c->mod[L + j] = p[j];
    for (int i = 0; i < L + K; i++) { if (c->mod[i] >= (1ULL << 62)) { free(c); return NULL; } c->bar[i] = barrett_make(c->mod[i]); }
    init_ntt_tables(c); init_encoder(c); init_keys(c);
    return c;
}
void orc_free(orc_ctx* c) {
    if (!c) return;
    free(c->psi); free(c->psip); free(c->ipsi); free(c->ipsip); free(c->s); free(c->s_ntt); free(c->pk);
    for (int i = 0; i < c->ngk; i++) free(c->gk[i].key);
    free(c->gk); free(c->rlk); free(c->rre); free(c->rim); free(c->rotgroup); free(c);
}

/* =====================================================================
 * 7. Encrypt / decrypt (Lattigo rlwe.Encryptor with a public key;
 *    encryptor.go:20-38).  Randomness: u ternary with h nonzeros, e0, e1 CBD,
 *    from streams indexed by enc_index.  Computed over Q + {p_0}, then ModDown.
 * ===================================================================== */
void orc_encrypt(const orc_ctx* c, const uint64_t* pt, int l, uint64_t enc, uint64_t* ct) {
    int N = c->N, nm = l + 2; int mi[MAXMOD];
    for (int i = 0; i <= l; i++) mi[i] = i;
    mi[l + 1] = c->L;
    i64* u = (i64*)xmalloc(sizeof(i64) * N); sample_ternary_hw(c->seed, ST_ENC_U(enc), N, c->h, u);
    u64* uq = (u64*)xmalloc(8 * (size_t)nm * N); poly_from_signed(c, u, mi, nm, uq); ntt_limbs(c, uq, mi, nm);
    u64* t0 = (u64*)xmalloc(8 * (size_t)nm * N); u64* t1 = (u64*)xmalloc(8 * (size_t)nm * N);
    int nqp = c->L + c->K;
    for (int j = 0; j < nm; j++) {
        int m = mi[j];
        for (int x = 0; x < N; x++) {
            size_t o = (size_t)j * N + x, ok = (size_t)m * N + x;
            t0[o] = mulmod_b(&c->bar[m], uq[o], c->pk[ok]);
            t1[o] = mulmod_b(&c->bar[m], uq[o], c->pk[(size_t)nqp * N + ok]);
        }
    }
    intt_limbs(c, t0, mi, nm); intt_limbs(c, t1, mi, nm);
    i64* e = (i64*)xmalloc(sizeof(i64) * N);
    u64* ep = (u64*)xmalloc(8 * (size_t)nm * N);
    sample_cbd(c->seed, ST_ENC_E0(enc), N, e); poly_from_signed(c, e, mi, nm, ep);
    for (int j = 0; j < nm; j++) for (int x = 0; x < N; x++) { size_t o = (size_t)j * N + x; t0[o] = addmod(t0[o], ep[o], c->mod[mi[j]]); }
    sample_cbd(c->seed, ST_ENC_E1(enc), N, e); poly_from_signed(c, e, mi, nm, ep);
    for (int j = 0; j < nm; j++) for (int x = 0; x < N; x++) { size_t o = (size_t)j * N + x; t1[o] = addmod(t1[o], ep[o], c->mod[mi[j]]); }
    u64* c0 = ct; u64* c1 = ct + (size_t)(l + 1) * N;
    mod_down_p0_coeff(c, l, t0, c0); mod_down_p0_coeff(c, l, t1, c1);
    int ql[MAXMOD]; q_list(c, l, ql);
    ntt_limbs(c, c0, ql, l + 1); ntt_limbs(c, c1, ql, l + 1);
    for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) { size_t o = (size_t)i * N + x; c0[o] = addmod(c0[o], pt[o], c->mod[i]); }
    free(u); free(uq); free(t0); free(t1); free(e); free(ep);
}
/* Seeded (secret-key) encryption, the compressed upload of the Cheddar
 * bindings (orion/backend/cheddar/ext/cheddar_pybind.cu:627-660): a is
 * expanded from the client's seed in the NTT domain, a[i][x] =
 * uniform(rand64(seed, ST_SEED_A, i*N + x)) mod q_i, so a server holding
 * only (b, seed) rebuilds it; b = -a*s + e + m with e CBD from the scheme
 * seed and encryption index. */
void orc_expand_seeded_a(const orc_ctx* c, int l, uint64_t seed, uint64_t* a) {
    int N = c->N;
    for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++)
        a[(size_t)i * N + x] = uniform_mod(orc_rand64(seed, ST_SEED_A, (u64)i * N + x), c->mod[i]);
}
void orc_encrypt_seeded(const orc_ctx* c, const uint64_t* pt, int l, uint64_t seed, uint64_t enc, uint64_t* ct) {
    int N = c->N; int ql[MAXMOD]; q_list(c, l, ql);
    u64* b = ct; u64* a = ct + (size_t)(l + 1) * N;
    orc_expand_seeded_a(c, l, seed, a);
    i64* e = (i64*)xmalloc(sizeof(i64) * N);
    sample_cbd(c->seed, ST_SEED_E(enc), N, e); poly_from_signed(c, e, ql, l + 1, b); ntt_limbs(c, b, ql, l + 1);
    for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) {
        size_t o = (size_t)i * N + x; u64 q = c->mod[i];
        b[o] = addmod(submod(b[o], mulmod_b(&c->bar[i], a[o], c->s_ntt[o]), q), pt[o], q);
    }
    free(e);
}
/* Multiplication by the imaginary unit: by the monomial X^(N/2) (it takes
 * the value i at every root zeta^(5^k)), key-free.  In the NTT domain slot j
 * holds the evaluation at psi^e, e = 2 brv(j) + 1, where X^(N/2) is
 * (psi^(N/2))^e = I^(e mod 4): I = psi^(N/2) for j < N/2, -I for j >= N/2. */
void orc_mul_i(const orc_ctx* c, const uint64_t* ct, int l, int npoly, uint64_t* out) {
    int N = c->N;
    for (int i = 0; i <= l; i++) {
        u64 q = c->mod[i];
        u64 I = c->psi[(size_t)i * N + 1], nI = q - I;  /* table slot brv(N/2) = 1 holds psi^(N/2) */
        for (int p = 0; p < npoly; p++) for (int x = 0; x < N; x++) {
            size_t o = ((size_t)p * (l + 1) + i) * N + x;
            out[o] = mulmod_b(&c->bar[i], ct[o], x < N / 2 ? I : nI);
        }
    }
}
void orc_decrypt(const orc_ctx* c, const uint64_t* ct, int l, uint64_t* pt) {
    int N = c->N; const u64* c0 = ct; const u64* c1 = ct + (size_t)(l + 1) * N;
    for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) {
        size_t o = (size_t)i * N + x;
        pt[o] = addmod(c0[o], mulmod_b(&c->bar[i], c1[o], c->s_ntt[o]), c->mod[i]);
    }
}

/* =====================================================================
 * 8. Evaluator: add, key switching, rotation, rescale
 * ===================================================================== */
void orc_add(const orc_ctx* c, const uint64_t* a, const uint64_t* b, int l, int npoly, uint64_t* out) {
    int N = c->N;
    for (int p = 0; p < npoly; p++) for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) {
        size_t o = ((size_t)p * (l + 1) + i) * N + x; out[o] = addmod(a[o], b[o], c->mod[i]);
    }
}
/* key limb offset of a QP limb k (position in a level-l QP poly) */
static inline int key_limb(const orc_ctx* c, int l, int k) { return k <= l ? k : c->L + (k - l - 1); }
/* (d0, d1) += sum_d digits[d] * key[d] over QP at level l (GadgetProductLazy body). */
static void gadget_mac(const orc_ctx* c, int l, const u64* digits, const u64* key, u64* d0, u64* d1) {
    int N = c->N, K = c->K, nqp = l + 1 + K, nm = c->L + K, dn = (l + 1 + K - 1) / K;
    #pragma omp parallel for num_threads(g_threads) schedule(static) if (g_threads > 1)
    for (int k = 0; k < nqp; k++) {
        int kl = key_limb(c, l, k); const barrett_t* B = &c->bar[kl]; u64 q = c->mod[kl];
        for (int x = 0; x < N; x++) {
            u64 a0 = 0, a1 = 0;
            for (int d = 0; d < dn; d++) {
                u64 dg = digits[((size_t)d * nqp + k) * N + x];
                const u64* kb = key + (size_t)d * 2 * nm * N;
                a0 = addmod(a0, mulmod_b(B, dg, kb[(size_t)kl * N + x]), q);
                a1 = addmod(a1, mulmod_b(B, dg, kb[(size_t)(nm + kl) * N + x]), q);
            }
            d0[(size_t)k * N + x] = a0; d1[(size_t)k * N + x] = a1;
        }
    }
}
static void mul_P_q(const orc_ctx* c, int l, const u64* in, u64* out) { /* out = P * in, Q limbs 0..l */
    int N = c->N;
    for (int i = 0; i <= l; i++) {
        u64 q = c->mod[i], P = 1;
        for (int j = 0; j < c->K; j++) P = orc_mulmod(P, c->mod[c->L + j] % q, q);
        for (int x = 0; x < N; x++) out[(size_t)i * N + x] = mulmod_b(&c->bar[i], in[(size_t)i * N + x], P);
    }
}
/* Lattigo Evaluator.Automorphism (evaluator.go:90-101 via ckks RotateNew):
 * GadgetProduct of c1 (decompose, key product, ModDown of both parts),
 * add c0, then the NTT-domain automorphism of both polynomials. */
void orc_automorphism_ct(orc_ctx* c, const uint64_t* ct, int l, uint64_t galel, uint64_t* out) {
    int N = c->N, K = c->K, nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
    const u64* key = orc_galois_key(c, galel);
    u64* digits = (u64*)xmalloc(8 * (size_t)dn * nqp * N);
    orc_decompose_modup(c, l, ct + (size_t)(l + 1) * N, digits);
    u64* d0 = (u64*)xmalloc(8 * (size_t)nqp * N); u64* d1 = (u64*)xmalloc(8 * (size_t)nqp * N);
    gadget_mac(c, l, digits, key, d0, d1);
    u64* t = (u64*)xmalloc(8 * (size_t)2 * (l + 1) * N);
    orc_mod_down(c, l, d0, t); orc_mod_down(c, l, d1, t + (size_t)(l + 1) * N);
    for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) { size_t o = (size_t)i * N + x; t[o] = addmod(t[o], ct[o], c->mod[i]); }
    uint32_t* idx = (uint32_t*)xmalloc(4 * (size_t)N); orc_automorphism_index(c, galel, idx);
    permute_limbs(c, t, out, 2 * (l + 1), idx);
    free(idx); free(t); free(d0); free(d1); free(digits);
}
void orc_rotate(orc_ctx* c, const uint64_t* ct, int l, int k, uint64_t* out) { orc_automorphism_ct(c, ct, l, orc_galois_element(c, k), out); }

/* Lattigo ckks Evaluator.Mul(ct, pt) (MulPlaintext, evaluator.go:274-295):
 * per-limb product of both parts with the plaintext at level min(lc, lp);
 * the output scale is the product of the scales (not rescaled). */
void orc_mul_plain(const orc_ctx* c, const uint64_t* ct, int lc, const uint64_t* pt, int lp, uint64_t* out) {
    int N = c->N, l = lc < lp ? lc : lp;
    for (int p = 0; p < 2; p++) for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) {
        size_t oc = ((size_t)p * (lc + 1) + i) * N + x, oo = ((size_t)p * (l + 1) + i) * N + x;
        out[oo] = mulmod_b(&c->bar[i], ct[oc], pt[(size_t)i * N + x]);
    }
}
typedef __int128 i128;
/* Residues of an integer constant k mod q. */
static u64 residue_i128(i128 k, u64 q) {
    if (k >= 0) return (u64)((u128)k % q);
    u64 m = (u64)((u128)(-(k + 1)) % q);  /* |k| - 1 without overflow */
    return negmod((m + 1) % q, q);
}
/* Lattigo's scaled real constant (bigComplexToRNSScalar at float64 encoding
 * precision): t = v * scale rounded to double, then +-0.5 (in double) and
 * truncated toward zero.  Returns 0 and sets *out when |t| < 2^125. */
static int scaled_constant128(double v, double scale, i128* out) {
    double t = v * scale;
    if (!(t < 42535295865117307932921825928971026432.0 && t > -42535295865117307932921825928971026432.0)) return -1;
    if (t > 0) t = t + 0.5; else if (t < 0) t = t - 0.5;
    *out = (i128)t;
    return 0;
}
int orc_scaled_constant(double v, double scale, int64_t* out) {
    i128 k;
    if (scaled_constant128(v, scale, &k) != 0 || k >= ((i128)1 << 62) || k <= -((i128)1 << 62)) return -1;
    *out = (int64_t)k;
    return 0;
}
static void mul_const128(const orc_ctx* c, const uint64_t* ct, int l, i128 k, uint64_t* out) {
    int N = c->N;
    for (int i = 0; i <= l; i++) {
        u64 kq = residue_i128(k, c->mod[i]);
        for (int p = 0; p < 2; p++) for (int x = 0; x < N; x++) {
            size_t o = ((size_t)p * (l + 1) + i) * N + x; out[o] = mulmod_b(&c->bar[i], ct[o], kq);
        }
    }
}
/* Evaluator.Mul(ct, int) (MulScalarInt, evaluator.go:188-205): every limb of
 * both parts times k mod q_i; the scale is unchanged. */
void orc_mul_int(const orc_ctx* c, const uint64_t* ct, int l, int64_t k, uint64_t* out) { mul_const128(c, ct, l, (i128)k, out); }
/* Evaluator.Mul(ct, float64) (MulScalarFloat, evaluator.go:208-225): an
 * integer-valued constant multiplies as an integer (scale unchanged);
 * otherwise the constant is scaled by q_l, rounded as above, and the output
 * scale is multiplied by q_l (the caller rescales).  Returns 1 when the
 * scale was multiplied by q_l, 0 when not, -1 when the constant is too large. */
int orc_mul_float(const orc_ctx* c, const uint64_t* ct, int l, double v, uint64_t* out) {
    i128 k;
    if (v < 4611686018427387904.0 && v > -4611686018427387904.0 && v == (double)(int64_t)v) {
        orc_mul_int(c, ct, l, (int64_t)v, out);
        return 0;
    }
    if (scaled_constant128(v, (double)c->mod[l], &k) != 0) return -1;
    mul_const128(c, ct, l, k, out);
    return 1;
}
/* Evaluator.Add(ct, float64) (AddScalar / SubScalar, evaluator.go:148-185):
 * the constant scaled by the ciphertext scale and rounded is added to (or
 * subtracted from) every NTT slot of part 0 in every limb. */
int orc_add_const(const orc_ctx* c, const uint64_t* ct, int l, double v, double scale, int sub, uint64_t* out) {
    int N = c->N; i128 k;
    if (scaled_constant128(v, scale, &k) != 0) return -1;
    if (out != ct) memcpy(out, ct, 8 * (size_t)2 * (l + 1) * N);
    for (int i = 0; i <= l; i++) {
        u64 q = c->mod[i], kq = residue_i128(k, q);
        for (int x = 0; x < N; x++) {
            size_t o = (size_t)i * N + x; out[o] = sub ? submod(ct[o], kq, q) : addmod(ct[o], kq, q);
        }
    }
    return 0;
}
/* Evaluator.MulRelin (MulRelinCiphertext, evaluator.go:343-362): tensor
 * (d0, d1, d2) = (a0 b0, a0 b1 + a1 b0, a1 b1) at level l, then d2 is key
 * switched with the relinearization key (decompose, key product, ModDown of
 * both parts) and added to (d0, d1).  The output scale is the product. */
void orc_mul_relin(orc_ctx* c, const uint64_t* a, const uint64_t* b, int l, uint64_t* out) {
    int N = c->N, K = c->K, nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
    size_t ps = (size_t)(l + 1) * N;
    u64* d2 = (u64*)xmalloc(8 * ps);
    for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) {
        size_t o = (size_t)i * N + x; const barrett_t* B = &c->bar[i]; u64 q = c->mod[i];
        out[o] = mulmod_b(B, a[o], b[o]);
        out[ps + o] = addmod(mulmod_b(B, a[o], b[ps + o]), mulmod_b(B, a[ps + o], b[o]), q);
        d2[o] = mulmod_b(B, a[ps + o], b[ps + o]);
    }
    const u64* rlk = orc_relin_key(c);
    u64* digits = (u64*)xmalloc(8 * (size_t)dn * nqp * N);
    orc_decompose_modup(c, l, d2, digits);
    u64* e0 = (u64*)xmalloc(8 * (size_t)nqp * N); u64* e1 = (u64*)xmalloc(8 * (size_t)nqp * N);
    gadget_mac(c, l, digits, rlk, e0, e1);
    u64* t = (u64*)xmalloc(8 * 2 * ps);
    orc_mod_down(c, l, e0, t); orc_mod_down(c, l, e1, t + ps);
    orc_add(c, out, t, l, 2, out);
    free(d2); free(digits); free(e0); free(e1); free(t);
}

/* Polynomial evaluation (EvaluatePolynomial, polyeval.go:62-84, monomial
 * basis of GenerateMonomial, polyeval.go:37-47), degree <= 3 at depth
 * ceil(log2(degree + 1)) (orion/nn/activation.py:22-28), the output scale
 * set to out_scale as Lattigo sets its target scale:
 *   d = 0: X*0 + c0                                       (level l)
 *   d = 1: Rescale(X * K1) + c0, K1 = round(c1 * So q_l / s)    (l-1)
 *   d = 2, 3: with X2 = Rescale(MulRelin(X, X)) (scale s^2 / q_l),
 *     B = Rescale(X * K3) + c2 at scale sB = So q_{l-1} / scale(X2),
 *         K3 = round(c3 * sB q_l / s);
 *     P = Rescale(MulRelin(X2, B))                              (l-2, So)
 *     A = Rescale(X * K1) dropped to l-2, + c0                  (l-2, So)
 *     out = P + A.
 * Constants are added as round(c * scale) (orc_add_const).  Returns the
 * output level, or -1 on an unsupported degree or too few levels. */
static void drop_to(const orc_ctx* c, const u64* ct, int l, int nl, u64* out) {
    size_t N = (size_t)c->N;
    for (int p = 0; p < 2; p++) memcpy(out + (size_t)p * (nl + 1) * N, ct + (size_t)p * (l + 1) * N, 8 * (size_t)(nl + 1) * N);
}
int orc_eval_poly(orc_ctx* c, const uint64_t* x, int l, double s, const double* coef, int d, double so, uint64_t* out) {
    int N = c->N;
    size_t ps = (size_t)N;
    while (d > 0 && coef[d] == 0.0) d--;
    if (d > 3 || d < 0) return -1;
    if (d == 0) {
        u64* z = (u64*)xmalloc(8 * 2 * (l + 1) * ps);
        orc_mul_int(c, x, l, 0, z);
        int r = orc_add_const(c, z, l, coef[0], so, 0, out);
        free(z);
        return r == 0 ? l : -1;
    }
    if (l < (d == 1 ? 1 : 2)) return -1;
    i128 k1;
    /* A = Rescale(X * K1) (+ c0 when d == 1) */
    if (scaled_constant128(coef[1], so * (double)c->mod[l] / s, &k1) != 0) return -1;
    u64* t = (u64*)xmalloc(8 * 2 * (l + 1) * ps);
    u64* A = (u64*)xmalloc(8 * 2 * l * ps);
    mul_const128(c, x, l, k1, t);
    orc_rescale(c, t, l, A);
    if (d == 1) {
        int r = orc_add_const(c, A, l - 1, coef[0], so, 0, out);
        free(t); free(A);
        return r == 0 ? l - 1 : -1;
    }
    double s2 = s * s / (double)c->mod[l];
    double sB = so * (double)c->mod[l - 1] / s2;
    double c3 = d == 3 ? coef[3] : 0.0;
    i128 k3;
    if (scaled_constant128(c3, sB * (double)c->mod[l] / s, &k3) != 0) { free(t); free(A); return -1; }
    u64* sq = (u64*)xmalloc(8 * 2 * (l + 1) * ps);
    u64* X2 = (u64*)xmalloc(8 * 2 * l * ps);
    orc_mul_relin(c, x, x, l, sq);
    orc_rescale(c, sq, l, X2);
    u64* B = (u64*)xmalloc(8 * 2 * l * ps);
    mul_const128(c, x, l, k3, t);
    orc_rescale(c, t, l, B);
    if (orc_add_const(c, B, l - 1, coef[2], sB, 0, B) != 0) { free(t); free(A); free(sq); free(X2); free(B); return -1; }
    u64* PB = (u64*)xmalloc(8 * 2 * l * ps);
    orc_mul_relin(c, X2, B, l - 1, PB);
    orc_rescale(c, PB, l - 1, out);
    u64* A2 = (u64*)xmalloc(8 * 2 * (l - 1) * ps);
    drop_to(c, A, l - 1, l - 2, A2);
    int r = orc_add_const(c, A2, l - 2, coef[0], so, 0, A2);
    orc_add(c, out, A2, l - 2, 2, out);
    free(t); free(A); free(sq); free(X2); free(B); free(PB); free(A2);
    return r == 0 ? l - 2 : -1;
}


/* Lattigo ring.DivRoundByLastModulusNTT (ckks Rescale, evaluator.go:131-146):
 * u = (iNTT(x_l) + q_l>>1) mod q_l; out_i = (x_i - NTT_i(u - q_l>>1)) * q_l^-1. */
void orc_rescale(const orc_ctx* c, const uint64_t* ct, int l, uint64_t* out) {
    int N = c->N; u64 ql = c->mod[l], half = ql >> 1;
    u64* u = (u64*)xmalloc(8 * (size_t)N); u64* t = (u64*)xmalloc(8 * (size_t)N);
    for (int p = 0; p < 2; p++) {
        const u64* x = ct + (size_t)p * (l + 1) * N; u64* o = out + (size_t)p * l * N;
        memcpy(u, x + (size_t)l * N, 8 * (size_t)N); orc_intt(c, l, u);
        for (int j = 0; j < N; j++) u[j] = addmod(u[j], half, ql);
        for (int i = 0; i < l; i++) {
            u64 q = c->mod[i], hq = half % q, inv = invmod_prime(ql % q, q);
            for (int j = 0; j < N; j++) t[j] = submod(u[j] % q, hq, q);
            orc_ntt(c, i, t);
            for (int j = 0; j < N; j++) o[(size_t)i * N + j] = mulmod_b(&c->bar[i], submod(x[(size_t)i * N + j], t[j], q), inv);
        }
    }
    free(u); free(t);
}

/* =====================================================================
 * 9. Linear transform (Lattigo circuits/ckks/lintrans; lineartransform.go:36-128)
 * ===================================================================== */
struct orc_lt {
    int level, slots, N1, nplain, ngiant, naive;
    int* plain_idx; u64** plain;     /* QP polys at level, NTT domain */
    int* giant; int* nbaby; int** baby;  /* BSGS index, giant keys sorted, babies sorted */
    int nrot2; int* rot2;                /* sorted distinct baby indices */
    int nrot1; int* rot1;                /* sorted distinct giant indices */
};
static int cmp_int(const void* a, const void* b) { int x = *(const int*)a, y = *(const int*)b; return (x > y) - (x < y); }
static int uniq_sorted(int* v, int n) { if (!n) return 0; qsort(v, n, sizeof(int), cmp_int); int m = 1; for (int i = 1; i < n; i++) if (v[i] != v[m - 1]) v[m++] = v[i]; return m; }
/* BSGSIndex: giant = ((rot/N1)*N1) & (slots-1), baby = rot & (N1-1) */
static void bsgs_index(const int* diags, int nd, int slots, int N1, int* nrot1, int* rot1, int* nrot2, int* rot2) {
    for (int i = 0; i < nd; i++) { int r = diags[i] & (slots - 1); rot1[i] = ((r / N1) * N1) & (slots - 1); rot2[i] = r & (N1 - 1); }
    *nrot1 = uniq_sorted(rot1, nd); *nrot2 = uniq_sorted(rot2, nd);
}
/* FindBestBSGSRatio: first N1 (powers of two) whose baby/giant count ratio
 * reaches 2^logMaxRatio; N1/2 if it overshoots. */
static int find_best_bsgs_ratio(const int* diags, int nd, int maxN, int logMaxRatio) {
    double maxRatio = (double)(1 << logMaxRatio);
    int* r1 = (int*)xmalloc(sizeof(int) * (nd + 1)); int* r2 = (int*)xmalloc(sizeof(int) * (nd + 1));
    for (int N1 = 1; N1 < maxN; N1 <<= 1) {
        int n1, n2; bsgs_index(diags, nd, maxN, N1, &n1, r1, &n2, r2);
        double nbN1 = (double)(n1 - 1), nbN2 = (double)(n2 - 1);
        double ratio = nbN2 / nbN1;
        if (ratio == maxRatio) { free(r1); free(r2); return N1; }
        if (ratio > maxRatio) { free(r1); free(r2); return N1 / 2; }
    }
    free(r1); free(r2);
    return 1;
}
static int lt_find(const orc_lt* t, int di) { for (int i = 0; i < t->nplain; i++) if (t->plain_idx[i] == di) return i; return -1; }

orc_lt* orc_lt_new(orc_ctx* c, const int* idx, int nidx, const float* data, int level, float bsgs_ratio) {
    int N = c->N, slots = N / 2, K = c->K, nqp = level + 1 + K;
    orc_lt* t = (orc_lt*)xcalloc(sizeof(orc_lt));
    t->level = level; t->slots = slots;
    int logratio = (int)log((double)bsgs_ratio); /* lineartransform.go:67: natural log, truncated */
    double scale = (double)c->mod[level];       /* lineartransform.go:64: Scale = Q[level] */
    int* keys = (int*)xmalloc(sizeof(int) * nidx);
    for (int i = 0; i < nidx; i++) keys[i] = idx[i];
    double* buf = (double*)xmalloc(sizeof(double) * slots);
    t->plain_idx = (int*)xmalloc(sizeof(int) * nidx); t->plain = (u64**)xcalloc(sizeof(u64*) * nidx);
    int* r1 = (int*)xmalloc(sizeof(int) * (nidx + 1)); int* r2 = (int*)xmalloc(sizeof(int) * (nidx + 1));
    if (logratio < 0) {
        t->naive = 1; t->N1 = 0;
        for (int i = 0; i < nidx; i++) {
            int di = keys[i] < 0 ? keys[i] + slots : keys[i];
            for (int k = 0; k < slots; k++) buf[k] = (double)data[(size_t)i * slots + k];
            t->plain_idx[t->nplain] = di; t->plain[t->nplain] = (u64*)xmalloc(8 * (size_t)nqp * N);
            orc_encode_f64(c, buf, slots, level, scale, 1, t->plain[t->nplain]); t->nplain++;
        }
        bsgs_index(keys, nidx, slots, slots, &t->nrot1, r1, &t->nrot2, r2);
        t->rot1 = r1; t->rot2 = r2;
    } else {
        int N1 = find_best_bsgs_ratio(keys, nidx, slots, logratio); t->N1 = N1;
        bsgs_index(keys, nidx, slots, N1, &t->nrot1, r1, &t->nrot2, r2);
        t->rot1 = r1; t->rot2 = r2;
        t->ngiant = t->nrot1; t->giant = (int*)xmalloc(sizeof(int) * t->ngiant);
        t->nbaby = (int*)xcalloc(sizeof(int) * t->ngiant); t->baby = (int**)xmalloc(sizeof(int*) * t->ngiant);
        for (int g = 0; g < t->ngiant; g++) { t->giant[g] = r1[g]; t->baby[g] = (int*)xmalloc(sizeof(int) * nidx); }
        for (int i = 0; i < nidx; i++) {
            int r = keys[i] & (slots - 1); int j = ((r / N1) * N1) & (slots - 1); int b = r & (N1 - 1);
            for (int g = 0; g < t->ngiant; g++) if (t->giant[g] == j) { t->baby[g][t->nbaby[g]++] = b; break; }
        }
        for (int g = 0; g < t->ngiant; g++) t->nbaby[g] = uniq_sorted(t->baby[g], t->nbaby[g]);
        /* the plaintext list (diagonal, source row, pre-rotation) in group order,
         * then the encodings, independent of each other, in parallel */
        int* srcs = (int*)xmalloc(sizeof(int) * (nidx + 1)); int* rotp = (int*)xmalloc(sizeof(int) * (nidx + 1));
        for (int g = 0; g < t->ngiant; g++) {
            int j = t->giant[g]; int rot = (-j) & (slots - 1);
            for (int bi = 0; bi < t->nbaby[g]; bi++) {
                int di = j + t->baby[g][bi], src = -1;
                for (int i = 0; i < nidx; i++) if (keys[i] == di || keys[i] == di - slots) { src = i; break; }
                if (src < 0) die("lintrans: diagonal missing");
                t->plain_idx[t->nplain] = di; srcs[t->nplain] = src; rotp[t->nplain] = rot;
                t->plain[t->nplain] = (u64*)xmalloc(8 * (size_t)nqp * N); t->nplain++;
            }
        }
        #pragma omp parallel num_threads(g_threads) if (g_threads > 1 && t->nplain > 1)
        {
            double* vb = (double*)xmalloc(sizeof(double) * slots);
            #pragma omp for schedule(dynamic, 1)
            for (int pi = 0; pi < t->nplain; pi++) {
                /* utils.RotateSliceAllocFree(v, rot): buf[k] = v[(k + rot) mod slots] */
                for (int k = 0; k < slots; k++) vb[k] = (double)data[(size_t)srcs[pi] * slots + ((k + rotp[pi]) & (slots - 1))];
                orc_encode_f64(c, vb, slots, level, scale, 1, t->plain[pi]);
            }
            free(vb);
        }
        free(srcs); free(rotp);
    }
    free(keys); free(buf);
    return t;
}
void orc_lt_free(orc_lt* t) {
    if (!t) return;
    for (int i = 0; i < t->nplain; i++) free(t->plain[i]);
    free(t->plain); free(t->plain_idx);
    for (int g = 0; g < t->ngiant; g++) free(t->baby[g]);
    free(t->baby); free(t->nbaby); free(t->giant); free(t->rot1); free(t->rot2); free(t);
}
int orc_lt_n1(const orc_lt* t) { return t->N1; }
int orc_lt_level(const orc_lt* t) { return t->level; }
int orc_lt_num_plaintexts(const orc_lt* t) { return t->nplain; }
int orc_lt_plaintext_index(const orc_lt* t, int i) { return t->plain_idx[i]; }
int orc_lt_num_giant(const orc_lt* t) { return t->ngiant; }
const uint64_t* orc_lt_plaintext(const orc_lt* t, int di) { int i = lt_find(t, di); return i < 0 ? NULL : t->plain[i]; }
/* GaloisElements (lineartransform.go:115-122): naive -> every nonzero
 * diagonal; BSGS -> giant and baby rotation sets (distinct, giant first,
 * both sorted).  The caller maps each rotation k to 5^k mod 2N. */
static int lt_rotations(const orc_lt* t, int* rots) {
    int n = 0;
    if (t->naive) { for (int i = 0; i < t->nrot2; i++) rots[n++] = t->rot2[i]; return n; }
    for (int i = 0; i < t->nrot1; i++) rots[n++] = t->rot1[i];
    for (int i = 0; i < t->nrot2; i++) { int dup = 0; for (int k = 0; k < n; k++) if (rots[k] == t->rot2[i]) dup = 1; if (!dup) rots[n++] = t->rot2[i]; }
    return n;
}
int orc_lt_rotations(const orc_lt* t, int* out) { return lt_rotations(t, out); }

/* plaintext limb k of a QP poly evaluated at level l, stored at level t->level */
static inline const u64* pt_limb(const orc_ctx* c, const orc_lt* t, const u64* pt, int l, int k) {
    int pos = k <= l ? k : (t->level + 1) + (k - l - 1);
    (void)c; return pt + (size_t)pos * c->N;
}
/* hoisted automorphism in QP (AutomorphismHoistedLazy): (sigma(d0 + P c0), sigma(d1)) */
static void hoisted_rot(orc_ctx* c, int l, const u64* digits, const u64* Pc0, u64 galel, u64* r0, u64* r1) {
    int N = c->N, nqp = l + 1 + c->K;
    u64* d0 = (u64*)xmalloc(8 * (size_t)nqp * N); u64* d1 = (u64*)xmalloc(8 * (size_t)nqp * N);
    gadget_mac(c, l, digits, orc_galois_key(c, galel), d0, d1);
    for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) { size_t o = (size_t)i * N + x; d0[o] = addmod(d0[o], Pc0[o], c->mod[i]); }
    uint32_t* idx = (uint32_t*)xmalloc(4 * (size_t)N); orc_automorphism_index(c, galel, idx);
    permute_limbs(c, d0, r0, nqp, idx); permute_limbs(c, d1, r1, nqp, idx);
    free(idx); free(d0); free(d1);
}
static inline u64 qp_mod(const orc_ctx* c, int l, int k) { return c->mod[key_limb(c, l, k)]; }
static inline const barrett_t* qp_bar(const orc_ctx* c, int l, int k) { return &c->bar[key_limb(c, l, k)]; }

/* MultiplyByDiagMatrixBSGS restated: one decomposition of c1; hoisted baby
 * rotations in QP; per giant group the inner sum in QP (baby 0 uses P*c);
 * for j != 0 ModDown of the c1-part, key switch of it, add the c0-part,
 * automorphism and accumulate in QP; one final ModDown of both parts. */
static void lt_eval_bsgs(orc_ctx* c, const orc_lt* t, const u64* ct, int ct_level, int g0, int g1, u64* acc, int final_moddown, u64* out) {
    int N = c->N, K = c->K;
    int l = ct_level < t->level ? ct_level : t->level;
    int nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
    const u64* c0 = ct; const u64* c1 = ct + (size_t)(ct_level + 1) * N;
    u64* digits = (u64*)xmalloc(8 * (size_t)dn * nqp * N);
    orc_decompose_modup(c, l, c1, digits);
    u64* Pc0 = (u64*)xmalloc(8 * (size_t)(l + 1) * N); u64* Pc1 = (u64*)xmalloc(8 * (size_t)(l + 1) * N);
    mul_P_q(c, l, c0, Pc0); mul_P_q(c, l, c1, Pc1);
    /* baby rotations */
    u64** R0 = (u64**)xcalloc(sizeof(u64*) * t->N1); u64** R1 = (u64**)xcalloc(sizeof(u64*) * t->N1);
    for (int bi = 0; bi < t->nrot2; bi++) {
        int b = t->rot2[bi]; if (b == 0) continue;
        R0[b] = (u64*)xmalloc(8 * (size_t)nqp * N); R1[b] = (u64*)xmalloc(8 * (size_t)nqp * N);
        hoisted_rot(c, l, digits, Pc0, orc_galois_element(c, b), R0[b], R1[b]);
    }
    u64* tmp0 = (u64*)xmalloc(8 * (size_t)nqp * N); u64* tmp1 = (u64*)xmalloc(8 * (size_t)nqp * N);
    u64* e0 = (u64*)xmalloc(8 * (size_t)nqp * N); u64* e1 = (u64*)xmalloc(8 * (size_t)nqp * N);
    u64* t1q = (u64*)xmalloc(8 * (size_t)(l + 1) * N);
    u64* dg2 = (u64*)xmalloc(8 * (size_t)dn * nqp * N);
    uint32_t* idx = (uint32_t*)xmalloc(4 * (size_t)N);
    u64* acc0 = acc; u64* acc1 = acc + (size_t)nqp * N;
    memset(acc, 0, 8 * (size_t)2 * nqp * N);
    for (int g = g0; g < g1 && g < t->ngiant; g++) {
        int j = t->giant[g];
        memset(tmp0, 0, 8 * (size_t)nqp * N); memset(tmp1, 0, 8 * (size_t)nqp * N);
        for (int bi = 0; bi < t->nbaby[g]; bi++) {
            int b = t->baby[g][bi];
            const u64* pt = orc_lt_plaintext(t, j + b);
            int nk = b == 0 ? l + 1 : nqp;
            #pragma omp parallel for num_threads(g_threads) schedule(static) if (g_threads > 1)
            for (int k = 0; k < nk; k++) {
                const u64* pl = pt_limb(c, t, pt, l, k); const barrett_t* B = qp_bar(c, l, k); u64 q = B->q;
                const u64* s0 = b == 0 ? Pc0 + (size_t)k * N : R0[b] + (size_t)k * N;
                const u64* s1 = b == 0 ? Pc1 + (size_t)k * N : R1[b] + (size_t)k * N;
                u64* o0 = tmp0 + (size_t)k * N; u64* o1 = tmp1 + (size_t)k * N;
                for (int x = 0; x < N; x++) {
                    o0[x] = addmod(o0[x], mulmod_b(B, pl[x], s0[x]), q);
                    o1[x] = addmod(o1[x], mulmod_b(B, pl[x], s1[x]), q);
                }
            }
        }
        if (j != 0) {
            orc_mod_down(c, l, tmp1, t1q);
            orc_decompose_modup(c, l, t1q, dg2);
            gadget_mac(c, l, dg2, orc_galois_key(c, orc_galois_element(c, j)), e0, e1);
            for (int k = 0; k < nqp; k++) { u64 q = qp_mod(c, l, k); for (int x = 0; x < N; x++) { size_t o = (size_t)k * N + x; e0[o] = addmod(e0[o], tmp0[o], q); } }
            orc_automorphism_index(c, orc_galois_element(c, j), idx);
            for (int k = 0; k < nqp; k++) {
                u64 q = qp_mod(c, l, k);
                for (int x = 0; x < N; x++) {
                    size_t o = (size_t)k * N + x, src = (size_t)k * N + idx[x];
                    acc0[o] = addmod(acc0[o], e0[src], q); acc1[o] = addmod(acc1[o], e1[src], q);
                }
            }
        } else {
            for (int k = 0; k < nqp; k++) { u64 q = qp_mod(c, l, k); for (int x = 0; x < N; x++) { size_t o = (size_t)k * N + x; acc0[o] = addmod(acc0[o], tmp0[o], q); acc1[o] = addmod(acc1[o], tmp1[o], q); } }
        }
    }
    if (final_moddown) { orc_mod_down(c, l, acc0, out); orc_mod_down(c, l, acc1, out + (size_t)(l + 1) * N); }
    for (int b = 0; b < t->N1; b++) { free(R0[b]); free(R1[b]); }
    free(R0); free(R1); free(tmp0); free(tmp1); free(e0); free(e1); free(t1q); free(dg2); free(idx);
    free(digits); free(Pc0); free(Pc1);
}
/* MultiplyByDiagMatrix (naive, N1 = 0): hoisted rotation per nonzero diagonal,
 * products summed in QP, ModDown, then the k = 0 diagonal times c added in Q. */
static void lt_eval_naive(orc_ctx* c, const orc_lt* t, const u64* ct, int ct_level, u64* out) {
    int N = c->N, K = c->K;
    int l = ct_level < t->level ? ct_level : t->level;
    int nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
    const u64* c0 = ct; const u64* c1 = ct + (size_t)(ct_level + 1) * N;
    u64* digits = (u64*)xmalloc(8 * (size_t)dn * nqp * N);
    orc_decompose_modup(c, l, c1, digits);
    u64* Pc0 = (u64*)xmalloc(8 * (size_t)(l + 1) * N); mul_P_q(c, l, c0, Pc0);
    u64* a0 = (u64*)xcalloc(8 * (size_t)nqp * N); u64* a1 = (u64*)xcalloc(8 * (size_t)nqp * N);
    u64* r0 = (u64*)xmalloc(8 * (size_t)nqp * N); u64* r1 = (u64*)xmalloc(8 * (size_t)nqp * N);
    int has0 = 0;
    for (int i = 0; i < t->nplain; i++) {
        int k = t->plain_idx[i] & (t->slots - 1);
        if (k == 0) { has0 = 1; continue; }
        hoisted_rot(c, l, digits, Pc0, orc_galois_element(c, k), r0, r1);
        const u64* pt = t->plain[i];
        for (int m = 0; m < nqp; m++) {
            const u64* pl = pt_limb(c, t, pt, l, m); const barrett_t* B = qp_bar(c, l, m);
            for (int x = 0; x < N; x++) {
                size_t o = (size_t)m * N + x;
                a0[o] = addmod(a0[o], mulmod_b(B, pl[x], r0[o]), B->q);
                a1[o] = addmod(a1[o], mulmod_b(B, pl[x], r1[o]), B->q);
            }
        }
    }
    orc_mod_down(c, l, a0, out); orc_mod_down(c, l, a1, out + (size_t)(l + 1) * N);
    if (has0) {
        const u64* pt = orc_lt_plaintext(t, 0);
        for (int p = 0; p < 2; p++) {
            const u64* cp = p ? c1 : c0; u64* o = out + (size_t)p * (l + 1) * N;
            for (int i = 0; i <= l; i++) for (int x = 0; x < N; x++) {
                size_t oo = (size_t)i * N + x;
                o[oo] = addmod(o[oo], mulmod_b(&c->bar[i], pt[oo], cp[oo]), c->mod[i]);
            }
        }
    }
    free(digits); free(Pc0); free(a0); free(a1); free(r0); free(r1);
}
void orc_lt_eval(orc_ctx* c, const orc_lt* t, const uint64_t* ct, int ct_level, uint64_t* out) {
    if (t->naive) { lt_eval_naive(c, t, ct, ct_level, out); return; }
    int l = ct_level < t->level ? ct_level : t->level;
    u64* acc = (u64*)xmalloc(8 * (size_t)2 * (l + 1 + c->K) * c->N);
    lt_eval_bsgs(c, t, ct, ct_level, 0, t->ngiant, acc, 1, out);
    free(acc);
}
