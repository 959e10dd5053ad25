// runtime.hip -- host runtime and C ABI of the MI355X CKKS backend.
//
// One global scheme per process (as the Lattigo wrapper's `scheme`,
// orion/backend/lattigo/scheme.go:32), one HIP stream, ID-handle registries
// with lowest-free-id reuse (orion/backend/lattigo/minheap.go:27-98).  All
// polynomial arithmetic runs on the GPU through kernels.hip; the host does
// only parameter set-up, the encoder's float64 FFT, the decoder's CRT and
// sampling of the small ternary vectors.  Every entry point returns -1 (or an
// empty array) and records a message for GetLastError() instead of aborting.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <tuple>
#include <memory>
#include <mutex>
#include <queue>
#include <set>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "fpntt.h"
#include "hipckks.h"
#include "kernels.h"
#include "../../include/helrm_hip.h"

// Device scratch of RotateInto, the entry point that allocates nothing: its
// key switch takes every temporary from this array (96 MiB, enough for a
// rotation at N = 2^16 with 24 Q and 8 P limbs).  Each GPU holds its own copy
// from the library's load to the process end.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address): it uses the per-device address hipGetSymbolAddress returns.
constexpr size_t SCRATCH_WORDS = (size_t)96 << 17;
static __device__ __align__(256) uint64_t scratch[SCRATCH_WORDS];

namespace {

// ============================================================================
// errors
// ============================================================================
thread_local std::string g_err;
struct Error : std::runtime_error { using std::runtime_error::runtime_error; };
#define HCHECK(x)                                                                                   \
  do {                                                                                              \
    hipError_t e_ = (x);                                                                            \
    if (e_ != hipSuccess) throw Error(std::string("HIP error: ") + hipGetErrorString(e_) + " at " + #x); \
  } while (0)
#define REQUIRE(c, msg) do { if (!(c)) throw Error(msg); } while (0)

template <class F> int guard(F&& f) {
  try { return f(); } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// ============================================================================
// host number theory
// ============================================================================
u64 mulmod(u64 a, u64 b, u64 m) { return (u64)((u128)a * b % m); }
u64 powmod(u64 a, u64 e, u64 m) { u64 r = 1 % m; a %= m; while (e) { if (e & 1) r = mulmod(r, a, m); a = mulmod(a, a, m); e >>= 1; } return r; }
u64 invmod(u64 a, u64 p) { return powmod(a % p, p - 2, p); }
u64 invmod_odd(u64 a, u64 m) {  // gcd(a, m) = 1, m a power of two or odd
  i64 t = 0, nt = 1; u64 r = m, nr = a % m;
  while (nr) { u64 q = r / nr; i64 tt = t - (i64)q * nt; t = nt; nt = tt; u64 rr = r - q * nr; r = nr; nr = rr; }
  if (t < 0) t += (i64)m;
  return (u64)t;
}
u64 shoup(u64 w, u64 q) { return (u64)(((u128)w << 64) / q); }
bool is_prime(u64 n) {
  static const u64 B[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  if (n < 2) return false;
  for (u64 b : B) { if (n == b) return true; if (n % b == 0) return false; }
  u64 d = n - 1; int s = 0;
  while (!(d & 1)) { d >>= 1; s++; }
  for (u64 b : B) {
    u64 x = powmod(b, d, n);
    if (x == 1 || x == n - 1) continue;
    bool comp = true;
    for (int r = 1; r < s; r++) { x = mulmod(x, x, n); if (x == n - 1) { comp = false; break; } }
    if (comp) return false;
  }
  return true;
}
u64 gcd(u64 a, u64 b) { while (b) { u64 t = a % b; a = b; b = t; } return a; }
u64 pollard(u64 n) {
  if (n % 2 == 0) return 2;
  for (u64 c = 1;; c++) {
    u64 x = 2, y = 2, d = 1;
    auto f = [&](u64 v) { return (mulmod(v, v, n) + c) % n; };
    while (d == 1) { x = f(x); y = f(f(y)); d = gcd(x > y ? x - y : y - x, n); }
    if (d != n) return d;
  }
}
void factor(u64 n, std::vector<u64>& f) {
  if (n == 1) return;
  if (is_prime(n)) { if (std::find(f.begin(), f.end(), n) == f.end()) f.push_back(n); return; }
  for (u64 p = 2; p < 1000; p++)
    if (n % p == 0) { factor(p, f); while (n % p == 0) n /= p; factor(n, f); return; }
  u64 d = pollard(n);
  factor(d, f); factor(n / d, f);
}
u64 smallest_generator(u64 q) {
  std::vector<u64> f; factor(q - 1, f);
  for (u64 g = 2;; g++) {
    bool ok = true;
    for (u64 p : f) if (powmod(g, (q - 1) / p, q) == 1) { ok = false; break; }
    if (ok) return g;
  }
}
// NTT-friendly chain (rlwe.GenModuli): per bit size, candidates 2^b + 1 +- k*2N,
// 61-bit downstream only, others alternating starting upstream; Q first, then P.
void gen_primes(int logN, const std::vector<int>& lq, const std::vector<int>& lp, std::vector<u64>& q, std::vector<u64>& p) {
  struct G { u64 up, down; bool next_up; };
  std::map<int, G> gens;
  u64 nth = (u64)2 << logN;
  auto next = [&](int b) {
    REQUIRE(b >= 10 && b <= 61, "prime bit sizes must be in [10, 61]");
    auto it = gens.find(b);
    if (it == gens.end()) it = gens.emplace(b, G{((u64)1 << b) + 1, ((u64)1 << b) + 1, true}).first;
    G& g = it->second;
    bool up = b == 61 ? false : g.next_up;
    if (b != 61) g.next_up = !g.next_up;
    for (;;) {
      u64 c;
      if (up) { g.up += nth; c = g.up; } else { g.down -= nth; c = g.down; }
      if (is_prime(c)) return c;
    }
  };
  q.clear(); p.clear();
  for (int b : lq) q.push_back(next(b));
  for (int b : lp) p.push_back(next(b));
}
int brv(int x, int logn) { int r = 0; for (int i = 0; i < logn; i++) { r = (r << 1) | (x & 1); x >>= 1; } return r; }

// ============================================================================
// counter PRNG (same specification as the device one in kernels.hip)
// ============================================================================
inline u64 mix64(u64 z) {
  z ^= z >> 30; z *= 0xbf58476d1ce4e5b9ULL;
  z ^= z >> 27; z *= 0x94d049bb133111ebULL;
  z ^= z >> 31; return z;
}
inline u64 rand64(u64 seed, u64 stream, u64 ctr) {
  u64 k = mix64(seed + 0x9e3779b97f4a7c15ULL * (stream + 1));
  return mix64(k ^ (ctr * 0xd1b54a32d192ed03ULL + 0x8cb92ba72f3d8dd7ULL));
}
constexpr u64 ST_SK = 1, ST_PK_A = 2, ST_PK_E = 3;
inline u64 ST_GK_A(u64 g, u64 d) { return (4ULL << 56) | (g << 8) | d; }
inline u64 ST_GK_E(u64 g, u64 d) { return (5ULL << 56) | (g << 8) | d; }
inline u64 ST_ENC_U(u64 e) { return (6ULL << 56) | e; }
inline u64 ST_ENC_E0(u64 e) { return (7ULL << 56) | e; }
inline u64 ST_ENC_E1(u64 e) { return (8ULL << 56) | e; }
inline u64 ST_RLK_A(u64 d) { return (9ULL << 56) | d; }
inline u64 ST_RLK_E(u64 d) { return (10ULL << 56) | d; }
constexpr u64 ST_SEED_A = 11ULL << 56;
inline u64 ST_SEED_E(u64 e) { return (12ULL << 56) | e; }
// ternary vector with exactly h entries +-1 (partial Fisher-Yates)
std::vector<int8_t> ternary_hw(u64 seed, u64 stream, int N, int h) {
  std::vector<int> idx(N);
  for (int i = 0; i < N; i++) idx[i] = i;
  std::vector<int8_t> out(N, 0);
  if (h > N) h = N;
  for (int k = 0; k < h; k++) {
    u64 r = rand64(seed, stream, (u64)k);
    int j = k + (int)(((u128)r * (u64)(N - k)) >> 64);
    std::swap(idx[k], idx[j]);
    out[idx[k]] = (rand64(seed, stream, (1ULL << 32) + (u64)k) & 1) ? -1 : 1;
  }
  return out;
}

// ============================================================================
// device memory: size-bucketed cache (no hipFree on the hot path)
// ============================================================================
// Size-bucketed cache of device buffers, one free list per HIP stream of the
// scheme: a buffer returned while stream i is current is handed out again
// only to later work on stream i, which runs after everything stream i was
// given before (work of the other stream that touched the buffer must have
// been joined first -- JoinStream -- before it is freed on stream i).
// Every pointer handed out is in live_ until it comes back; put() of any
// other pointer (a second free, or a buffer released with its scheme) is
// refused instead of entering a free list, where it could be handed out twice.
struct Pool {
  static constexpr int NSTREAMS = 2;
  std::multimap<size_t, void*> free_[NSTREAMS];
  std::unordered_map<void*, size_t> size_;
  std::unordered_set<void*> live_;
  std::unordered_set<void*> user_;  // handed out by DeviceAlloc (released by DeleteScheme)
  size_t live = 0, cached = 0, peak = 0;
  int cur = 0;  // the scheme's current stream
  int forbid = 0;  // > 0 inside an entry point that allocates nothing: get() is an error
  void* get(size_t bytes) {
    REQUIRE(!forbid, "device allocation inside an entry point that allocates nothing");
    bytes = (bytes + 255) & ~(size_t)255;
    if (bytes == 0) bytes = 256;
    auto& fl = free_[cur];
    auto it = fl.find(bytes);
    if (it != fl.end()) {
      void* p = it->second; fl.erase(it); cached -= bytes; live += bytes; peak = std::max(peak, live);
      live_.insert(p);
      return p;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) { (void)hipGetLastError(); trim(); HCHECK(hipMalloc(&p, bytes)); }
    size_[p] = bytes; live += bytes; peak = std::max(peak, live);
    live_.insert(p);
    return p;
  }
  // returns false (and changes nothing) for a pointer that is not live
  bool put(void* p) {
    if (!p) return true;
    if (!live_.erase(p)) return false;
    const size_t b = size_.at(p);
    free_[cur].emplace(b, p); live -= b; cached += b;
    return true;
  }
  void trim() {
    (void)hipDeviceSynchronize();
    for (auto& fl : free_) {
      for (auto& kv : fl) { (void)hipFree(kv.second); size_.erase(kv.second); }
      fl.clear();
    }
    cached = 0;
  }
  void release_all() {
    (void)hipDeviceSynchronize();
    for (auto& kv : size_) (void)hipFree(kv.first);
    for (auto& fl : free_) fl.clear();
    size_.clear(); live_.clear(); user_.clear(); live = cached = 0; cur = 0;
  }
};
Pool* g_pool = nullptr;

// Device address of `scratch` per device, taken once per device when a
// scheme is built on it (with that device current).
// A failure is kept per device and reported by RotateInto, so that the rest
// of the library works without the scratch array.
// Calls on different streams are ordered on the array: `ev` is recorded on
// the stream of the last call after its key switch, and a call on another
// stream waits for it first (hipStreamWaitEvent allocates nothing).
std::map<int, uint64_t*> g_scratch;
std::map<int, std::string> g_scratch_err;
struct ScratchUse { hipEvent_t ev = nullptr; hipStream_t last = nullptr; };
std::map<int, ScratchUse> g_scratch_use;
void init_scratch() {
  int dev = 0;
  HCHECK(hipGetDevice(&dev));
  if (g_scratch.count(dev)) return;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) {
    (void)hipGetLastError();
    g_scratch_err[dev] = std::string("device scratch has no address: ") + hipGetErrorString(e);
    return;
  }
  HCHECK(hipEventCreateWithFlags(&g_scratch_use[dev].ev, hipEventDisableTiming));
  g_scratch[dev] = static_cast<uint64_t*>(ptr);
  g_scratch_err.erase(dev);
}
ScratchUse& scratch_use() {
  int dev = 0;
  HCHECK(hipGetDevice(&dev));
  return g_scratch_use.at(dev);
}
uint64_t* scratch_ptr() {
  int dev = 0;
  HCHECK(hipGetDevice(&dev));
  auto it = g_scratch.find(dev);
  if (it != g_scratch.end()) return it->second;
  auto er = g_scratch_err.find(dev);
  throw Error(er != g_scratch_err.end() ? er->second : "device scratch not set up on this device: build a scheme on it first");
}

template <class T> struct DevArray {
  T* p = nullptr; size_t n = 0;
  DevArray() = default;
  explicit DevArray(size_t count) : n(count) { if (count) p = (T*)g_pool->get(count * sizeof(T)); }
  DevArray(const DevArray&) = delete;
  DevArray& operator=(const DevArray&) = delete;
  DevArray(DevArray&& o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
  DevArray& operator=(DevArray&& o) noexcept { if (this != &o) { reset(); p = o.p; n = o.n; o.p = nullptr; o.n = 0; } return *this; }
  ~DevArray() { reset(); }
  void reset() { if (p && g_pool) (void)g_pool->put(p); p = nullptr; n = 0; }
  size_t bytes() const { return n * sizeof(T); }
};
using DU64 = DevArray<u64>;

// ============================================================================
// scheme objects
// ============================================================================
struct IdHeap {  // lowest free id first
  int next = 0;
  std::priority_queue<int, std::vector<int>, std::greater<int>> freed;
  int take() { if (!freed.empty()) { int v = freed.top(); freed.pop(); return v; } return next++; }
  void give(int v) { freed.push(v); }
};
struct Plain { int level; double scale; int logslots; DU64 d; };      // [level+1][N]
struct Cipher { int level; double scale; int logslots; DU64 d; };     // [2][level+1][N]
struct LinTrans {
  int level = 0, N1 = 0, slots = 0;
  bool naive = false;
  std::vector<int> keys;                 // diagonal indices as given
  std::vector<int> rot1, rot2;           // sorted giant / baby rotations
  std::vector<int> giant;                // giant rotation per group
  std::vector<std::vector<int>> baby;    // sorted babies per group
  std::vector<int> plain_idx;            // diagonal index of each stored plaintext
  DU64 diags;                            // [np][level+1+K][N], Montgomery form (packed: see below)
  // dense 16-baby transforms store their diagonals packed (rows of moduli
  // below 2^52 as 52-bit fields, PK_CHUNK dwords per 64 words): per row its
  // dword offset and 52 or 0 (plain), and the dwords of one diagonal
  bool packed = false;
  std::vector<uint32_t> pkrow;
  DevArray<uint32_t> d_pkrow;
  size_t pk_stride = 0;
  std::vector<char> resident;            // per stored plaintext: loaded (SerializeDiagonal / Remove drop it)
  DevArray<int> d_gpi, d_bzero, d_bslot;  // [ng][nbaby] plaintext index (absent: the zero plaintext); per-baby flags
  std::vector<int> gpi, bzero, bslot;     // host copies, checked before every diagonal-MAC launch
  bool dense = false;                     // every giant group holds every baby step
  double scale = 0;
  // device arrays of key / permutation pointers (baby and giant rotations), built on first use
  DevArray<const u64*> d_bkey, d_gkey; DevArray<const uint32_t*> d_bperm, d_gperm; DevArray<int> d_tg;
  DevArray<u64> d_bka, d_gka;  // [key][dnum] stream keys of the keys' a halves (used when every key was generated here)
  bool ptrs_ready = false;
};

struct BConvHost { int ns; BConvTable tab; DU64 hat, vS; DevArray<BConvTable> dtab; };

struct Timing { bool on = false; std::map<std::string, std::vector<std::pair<hipEvent_t, hipEvent_t>>> ev; std::map<std::string, std::pair<long, double>> acc; };

struct Scheme {
  int logN = 0, N = 0, L = 0, K = 0, dnum = 0, logscale = 0, h = 0;
  u64 seed = 0;
  std::vector<u64> mod;
  hipStream_t st = nullptr;  // the current stream: every public call is ordered on it
  // streams[0] is created with the scheme, streams[1] on the first SetStream(1);
  // both at the default priority
  hipStream_t streams[2] = {nullptr, nullptr};
  hipEvent_t join_ev[2] = {nullptr, nullptr};  // recorded on streams[i] by JoinStream(i)
  DevArray<ModC> d_mods;
  DU64 tw2, itw2, ninv, ninvp;  // interleaved (w, w') twiddle pairs [mod][N][2]
  DU64 twr2, itwr2;             // row-pass consecutive-round twiddles, lane-interleaved
  DevArray<FpC> fpc;            // float64 transform constants (moduli <= FP_QMAX)
  NttTables tw{};
  std::vector<ModC> hmods;
  // per-modulus constants (Shoup pairs indexed by modulus)
  DU64 pmod_w, pmod_wp, pinv_w, pinv_wp, p0inv_w, p0inv_wp, pmod_plain;
  DU64 rs_inv, rs_invp;  // [l][i] q_l^-1 mod q_i
  DU64 prs_inv, prs_invp;  // [l][i] (P q_l)^-1 mod q_i
  std::vector<u64> pinv_h, pinv_hp;  // [i] P^-1 mod q_i and its Shoup companion (host copies)
  // EvaluateLinearTransform returns the rescaled result (ModDown and rescale
  // fused), as backends that advertise lt_output_prerescaled do
  bool lt_prerescale = false;
  DU64 iu, iup, niu, niup;  // [mod] psi^(N/2) (a square root of -1), its negation, Shoup companions
  std::map<std::pair<int, int>, std::unique_ptr<BConvHost>> bconv;
  std::map<u64, DevArray<uint32_t>> perms, perm_invs;
  std::map<std::tuple<int, int, size_t>, std::unique_ptr<struct DigitRows>> digit_rows;
  // Galois keys this library generated (a halves a function of the seed, the
  // key's stream and the word's position, regenerated by the kernels); a
  // loaded key is read whole
  std::set<u64> seeded_gk;
  bool rlk_seeded = false;
  // keys
  bool has_sk = false, has_pk = false;
  std::vector<int8_t> s;
  DU64 sR, pkR;
  std::map<u64, std::unique_ptr<DU64>> gkeys;
  std::unique_ptr<DU64> rlk;  // relinearization key s^2 -> s
  std::set<u64> rot_keys, lt_keys;
  u64 enc_counter = 0;
  // registries
  IdHeap pt_ids, ct_ids, lt_ids, poly_ids;
  std::map<int, std::vector<double>> polys;  // monomial coefficients, lowest degree first
  std::map<int, std::unique_ptr<Plain>> pts;
  std::map<int, std::unique_ptr<Cipher>> cts;
  std::map<int, std::unique_ptr<LinTrans>> lts;
  // encoder
  std::vector<double> rre, rim;
  std::vector<int> rotgroup;
  DevArray<double> d_rre, d_rim;
  DevArray<int> d_rotgroup;
  Timing timing;
  bool encoder = false, encryptor = false, decryptor = false, evaluator = false, lteval = false;
  ~Scheme() {
    for (hipStream_t& x : streams)
      if (x) { (void)hipStreamSynchronize(x); (void)hipStreamDestroy(x); x = nullptr; }
    for (hipEvent_t& e : join_ev)
      if (e) { (void)hipEventDestroy(e); e = nullptr; }
  }
};
Scheme* S = nullptr;
u64 g_seed_override = 0;
bool g_seed_set = false;

Scheme& sch() { REQUIRE(S, "no scheme: call NewScheme first"); return *S; }
void sync() { HCHECK(hipStreamSynchronize(sch().st)); }
template <class T> void upload(T* d, const T* h, size_t n) { HCHECK(hipMemcpyAsync(d, h, n * sizeof(T), hipMemcpyHostToDevice, sch().st)); HCHECK(hipStreamSynchronize(sch().st)); }
template <class T> void download(T* h, const T* d, size_t n) { HCHECK(hipMemcpyAsync(h, d, n * sizeof(T), hipMemcpyDeviceToHost, sch().st)); HCHECK(hipStreamSynchronize(sch().st)); }
void d2d(void* dst, const void* src, size_t bytes) { if (bytes) HCHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, sch().st)); }
// batched strided copy of `words` u64 per batch entry (own kernel: one launch, 16 B per lane)
void copy_rows(u64* dst, size_t dstride, const u64* src, size_t sstride, size_t words, int batch) {
  launch_copy(dst, dstride, src, sstride, words, batch, sch().st);
}

RowMap rows_q(int l) { return RowMap{l + 1, l + 1, 0, 0, 0, 0}; }
RowMap rows_p() { Scheme& s = sch(); return RowMap{s.K, 0, 0, s.L, 0, 0}; }
RowMap rows_all() { Scheme& s = sch(); return RowMap{s.L + s.K, s.L + s.K, 0, 0, 0, 0}; }
inline int qp_mod(int l, int k) { Scheme& s = sch(); return k <= l ? k : s.L + (k - l - 1); }

void ntt(u64* d, size_t bstride, int batch, RowMap rm, bool fwd) { Scheme& s = sch(); launch_ntt(d, bstride, batch, rm, s.logN, fwd, s.tw, s.st); }
void ntt_oop(const u64* src, size_t sstride, u64* dst, size_t dstride, int batch, RowMap rm, bool fwd) {
  Scheme& s = sch();
  launch_ntt(src, sstride, dst, dstride, batch, rm, s.logN, fwd, s.tw, s.st);
}

// timing of named launches (HIP events on the scheme stream)
template <class F> void timed(const char* name, F&& f) {
  Scheme& s = sch();
  if (!s.timing.on) { f(); return; }
  hipEvent_t a, b;
  HCHECK(hipEventCreate(&a)); HCHECK(hipEventCreate(&b));
  HCHECK(hipEventRecord(a, s.st));
  f();
  HCHECK(hipEventRecord(b, s.st));
  s.timing.ev[name].push_back({a, b});
}
void timing_collect() {
  Scheme& s = sch();
  for (auto& kv : s.timing.ev) {
    for (auto& pr : kv.second) {
      HCHECK(hipEventSynchronize(pr.second));
      float ms = 0; HCHECK(hipEventElapsedTime(&ms, pr.first, pr.second));
      auto& a = s.timing.acc[kv.first]; a.first++; a.second += ms;
      (void)hipEventDestroy(pr.first); (void)hipEventDestroy(pr.second);
    }
  }
  s.timing.ev.clear();
}

// ============================================================================
// basis-conversion tables: src = moduli [s0, s1) (indices), all moduli as targets
// ============================================================================
BConvHost& bconv_table(int s0, int s1) {
  Scheme& s = sch();
  auto key = std::make_pair(s0, s1);
  auto it = s.bconv.find(key);
  if (it != s.bconv.end()) return *it->second;
  int ns = s1 - s0, nm = s.L + s.K;
  REQUIRE(ns >= 1 && ns <= HCK_MAXSRC, "basis conversion source too large");
  auto b = std::make_unique<BConvHost>();
  b->ns = ns;
  std::vector<u64> hat((size_t)nm * ns), vS((size_t)nm * (ns + 1));
  for (int i = 0; i < ns; i++) {
    u64 si = s.mod[s0 + i], pr = 1;
    for (int j = 0; j < ns; j++) if (j != i) pr = mulmod(pr, s.mod[s0 + j] % si, si);
    u64 hi = invmod(pr, si);
    b->tab.src[i] = BConvSrc{si, hi, shoup(hi, si), (double)si};
  }
  for (int m = 0; m < nm; m++) {
    u64 t = s.mod[m], R = s.hmods[m].rmod, Sm = 1;
    for (int j = 0; j < ns; j++) Sm = mulmod(Sm, s.mod[s0 + j] % t, t);
    for (int v = 0; v <= ns; v++) vS[(size_t)m * (ns + 1) + v] = mulmod((u64)v, Sm, t);
    for (int i = 0; i < ns; i++) {
      u64 pr = 1;
      for (int j = 0; j < ns; j++) if (j != i) pr = mulmod(pr, s.mod[s0 + j] % t, t);
      hat[(size_t)m * ns + i] = mulmod(pr, R, t);
    }
  }
  hat.resize(hat.size() + 8, 0);  // spare words: the 8-source kernel reads h[ns..7] (times zero) past the last row
  b->hat = DU64(hat.size()); upload(b->hat.p, hat.data(), hat.size());
  b->vS = DU64(vS.size()); upload(b->vS.p, vS.data(), vS.size());
  b->tab.hat = b->hat.p; b->tab.vS = b->vS.p; b->tab.rows_per_block = 8;
  b->dtab = DevArray<BConvTable>(1); upload(b->dtab.p, &b->tab, 1);
  auto& ref = *b;
  s.bconv[key] = std::move(b);
  return ref;
}

// The table of a source range that must already exist (built with the
// scheme for every digit split and for P -> Q): a lookup that allocates nothing.
BConvHost& bconv_table_cached(int s0, int s1) {
  Scheme& s = sch();
  auto it = s.bconv.find(std::make_pair(s0, s1));
  REQUIRE(it != s.bconv.end(), "basis conversion table missing");
  return *it->second;
}
// Every table a key switch at any level reads: each digit [dK, min(dK+K, l+1))
// of each level l, and the P -> Q extension of ModDown.
void prebuild_bconv_tables() {
  Scheme& s = sch();
  for (int l = 0; l < s.L; l++)
    for (int st0 = 0; st0 <= l; st0 += s.K) bconv_table(st0, std::min(st0 + s.K, l + 1));
  bconv_table(s.L, s.L + s.K);
}

const uint32_t* perm_for(u64 galel) {
  Scheme& s = sch();
  auto it = s.perms.find(galel);
  if (it != s.perms.end()) return it->second.p;
  std::vector<uint32_t> idx(s.N);
  u64 mask = 2 * (u64)s.N - 1;
  for (int i = 0; i < s.N; i++) {
    u64 e = 2 * (u64)brv(i, s.logN) + 1;
    u64 t = ((galel * e) & mask) - 1;
    idx[i] = (uint32_t)brv((int)(t >> 1), s.logN);
  }
  DevArray<uint32_t> d(s.N); upload(d.p, idx.data(), idx.size());
  const uint32_t* p = d.p;
  s.perms[galel] = std::move(d);
  return p;
}
// inverse of perm_for(galel): out[inv[p]] = in[p]
const uint32_t* perm_inv_for(u64 galel) {
  Scheme& s = sch();
  auto it = s.perm_invs.find(galel);
  if (it != s.perm_invs.end()) return it->second.p;
  std::vector<uint32_t> idx(s.N), inv(s.N);
  u64 mask = 2 * (u64)s.N - 1;
  for (int i = 0; i < s.N; i++) {
    u64 e = 2 * (u64)brv(i, s.logN) + 1;
    u64 t = ((galel * e) & mask) - 1;
    idx[i] = (uint32_t)brv((int)(t >> 1), s.logN);
  }
  for (int i = 0; i < s.N; i++) inv[idx[i]] = (uint32_t)i;
  DevArray<uint32_t> d(s.N); upload(d.p, inv.data(), inv.size());
  const uint32_t* p = d.p;
  s.perm_invs[galel] = std::move(d);
  return p;
}
// the inverse gather of an automorphism whose key exists (built with the key)
const uint32_t* perm_inv_cached(u64 galel) {
  auto it = sch().perm_invs.find(galel);
  REQUIRE(it != sch().perm_invs.end(), "automorphism table missing");
  return it->second.p;
}
u64 galois_element(int k) { Scheme& s = sch(); u64 M = 2 * (u64)s.N; return powmod(5, (u64)(i64)k & (M - 1), M); }

// ============================================================================
// key switching building blocks
// ============================================================================
// digits[b][d][nqp][N] from c1 (NTT, Q rows 0..l) of batch b (stride c1_bstride)
// The extended rows of every digit of a decomposition at level l for `batch`
// entries of stride dstride: {word offset, modulus} per limb, built once.
struct LimbRefH { int64_t off; int mod; int pad; };
struct DigitRows { DevArray<LimbRefH> list; int n = 0; };
const DigitRows& digit_rows(int l, int batch, size_t dstride) {
  Scheme& s = sch();
  const auto key = std::make_tuple(l, batch, dstride);
  auto it = s.digit_rows.find(key);
  if (it != s.digit_rows.end()) return *it->second;
  const int N = s.N, K = s.K, nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
  // modulus-major, so that consecutive limbs share their twiddle tables in L2
  std::vector<LimbRefH> v;
  for (int k = 0; k < nqp; k++)
    for (int b = 0; b < batch; b++)
      for (int d = 0; d < dn; d++) {
        const int st0 = d * K, en = std::min(st0 + K, l + 1);
        if (k < st0 || k >= en)
          v.push_back(LimbRefH{(int64_t)((size_t)b * dstride + ((size_t)d * nqp + k) * N), qp_mod(l, k), 0});
      }
  auto dr = std::make_unique<DigitRows>();
  dr->n = (int)v.size();
  dr->list = DevArray<LimbRefH>(v.size());
  upload(dr->list.p, v.data(), v.size());
  const DigitRows& ref = *dr;
  s.digit_rows[key] = std::move(dr);
  return ref;
}

// copy_own: also copy each digit's own rows (the key-product kernels can instead read them from c1)
// coef_ws: nullptr -> the coefficient-domain copy of c1 comes from the buffer
// cache; else batch * (l+1) * N device words the call may overwrite, and the
// forward transforms go per digit over a RowMap (nothing is allocated)
void decompose_modup(int l, const u64* c1, size_t c1_bstride, int batch, u64* digits, bool copy_own = true,
                     u64* coef_ws = nullptr) {
  Scheme& s = sch();
  const int N = s.N, K = s.K, nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
  const size_t dstride = (size_t)dn * nqp * N;
  DU64 coef_buf;
  if (!coef_ws) coef_buf = DU64((size_t)batch * (l + 1) * N);
  u64* coef = coef_ws ? coef_ws : coef_buf.p;
  ntt_oop(c1, c1_bstride, coef, (size_t)(l + 1) * N, batch, rows_q(l), false);
  // every digit's extension in one launch: targets are every QP row except the digit's own [st0, en)
  REQUIRE(dn <= HCK_MAXJOBS, "too many decomposition digits");
  BConvJobs jobs{};
  jobs.n = dn;
  for (int d = 0; d < dn; d++) {
    const int st0 = d * K, en = std::min(st0 + K, l + 1), ns = en - st0;
    jobs.j[d] = BConvJob{bconv_table_cached(st0, en).dtab.p, st0, ns, ns == 1 ? 1 : 0, 0, RowMap{nqp, l + 1, 0, s.L, st0, en},
                         (size_t)d * nqp * N};
  }
  launch_bconv(coef, (size_t)(l + 1) * N, jobs, digits, dstride, batch, s.d_mods.p, N, s.st);
  if (copy_own)
    for (int d = 0; d < dn; d++) {
      const int st0 = d * K, ns = std::min(st0 + K, l + 1) - st0;
      u64* D = digits + (size_t)d * nqp * N;
      copy_rows(D + (size_t)st0 * N, dstride, c1 + (size_t)st0 * N, c1_bstride, (size_t)ns * N, batch);
    }
  if (coef_ws) {
    // a digit's extended rows: every QP row but its own [st0, en)
    for (int d = 0; d < dn; d++) {
      const int st0 = d * K, en = std::min(st0 + K, l + 1);
      launch_ntt(digits + (size_t)d * nqp * N, dstride, batch, RowMap{nqp, l + 1, 0, s.L, st0, en}, s.logN, true, s.tw, s.st);
    }
    return;
  }
  // one forward transform over the extended rows of every digit of every batch entry
  const DigitRows& dr = digit_rows(l, batch, dstride);
  launch_ntt_list(digits, dr.list.p, dr.n, s.logN, true, s.tw, s.st);
}
// out[b] (Q rows, stride o_bstride) = ModDown(x[b]) (QP rows, stride x_bstride) [+ add[b<add_batches]],
// written through perm_inv (out[perm_inv[p]] takes position p; nullptr: identity)
// ws: nullptr -> temporaries from the buffer cache; else batch * (K + l + 1) * N
// device words the call may overwrite (nothing is allocated)
// acc: nullptr, or a buffer other than out whose words (at the output
// positions, batch stride o_bstride) are added to the result
void mod_down(int l, const u64* x, size_t x_bstride, int batch, u64* out, size_t o_bstride, const u64* add = nullptr,
              size_t a_bstride = 0, int add_batches = 0, const uint32_t* perm_inv = nullptr, u64* ws = nullptr,
              const u64* acc = nullptr) {
  Scheme& s = sch();
  const int N = s.N, K = s.K;
  DU64 pc_buf, ext_buf;
  if (!ws) { pc_buf = DU64((size_t)batch * K * N); ext_buf = DU64((size_t)batch * (l + 1) * N); }
  u64* pc = ws ? ws : pc_buf.p;
  u64* ext = ws ? ws + (size_t)batch * K * N : ext_buf.p;
  // P rows of x (rows l+1.. of each batch entry) -> coefficient domain in pc
  ntt_oop(x + (size_t)(l + 1) * N, x_bstride, pc, (size_t)K * N, batch, rows_p(), false);
  BConvHost& bt = bconv_table_cached(s.L, s.L + K);
  launch_bconv(pc, (size_t)K * N, K, bt.dtab.p, ext, (size_t)(l + 1) * N, batch, rows_q(l), s.d_mods.p, N, false, s.st);
  // forward transform of the extension fused with (x - ext) * P^-1 (+ add), gathered through perm
  launch_ntt_moddown(ext, (size_t)(l + 1) * N, batch, l, s.logN, x, x_bstride, out, o_bstride, add, a_bstride,
                     add_batches, perm_inv, s.pinv_w.p, s.pinv_wp.p, s.tw, s.st, acc, o_bstride);
}

// out[b] (Q rows 0..l-1, stride o_bstride) = Rescale(ModDown(x[b])) for the
// QP polynomials x[b] at level l, word for word what mod_down followed by
// rescale_ct computes: the ModDown result's row l is formed in the coefficient
// domain from the inverse transform of x's row l and the extension of [x]_P,
// the rescale's correction t is spread from it, and one forward transform of
// ext_i + P t_i ends in (x_i - NTT(ext_i + P t_i)) * (P q_l)^-1 -- the
// rescale's own inverse and forward transforms are not needed.
void mod_down_rescale(int l, const u64* x, size_t x_bstride, int batch, u64* out, size_t o_bstride) {
  Scheme& s = sch();
  const int N = s.N, K = s.K;
  REQUIRE(l >= 1, "cannot rescale: ciphertext already at level 0");
  DU64 pcq((size_t)batch * (K + 1) * N), ext((size_t)batch * (l + 1) * N);
  // rows l (q_l) and l+1.. (P) of x are consecutive: one inverse transform
  ntt_oop(x + (size_t)l * N, x_bstride, pcq.p, (size_t)(K + 1) * N, batch, RowMap{K + 1, 1, l, s.L, 0, 0}, false);
  BConvHost& bt = bconv_table(s.L, s.L + K);
  launch_bconv(pcq.p + N, (size_t)(K + 1) * N, K, bt.dtab.p, ext.p, (size_t)(l + 1) * N, batch, rows_q(l), s.d_mods.p, N, false,
               s.st);
  launch_moddown_rescale_spread(ext.p, (size_t)(l + 1) * N, pcq.p, (size_t)(K + 1) * N, l, s.mod[l] >> 1, s.pinv_h[l],
                                s.pinv_hp[l], s.pmod_w.p, s.pmod_wp.p, s.d_mods.p, N, batch, s.st);
  launch_ntt_moddown(ext.p, (size_t)(l + 1) * N, batch, l - 1, s.logN, x, x_bstride, out, o_bstride, nullptr, 0, 0, nullptr,
                     s.prs_inv.p + (size_t)l * s.L, s.prs_invp.p + (size_t)l * s.L, s.tw, s.st);
}

const u64* key_ptr(u64 galel, bool for_lt) {
  Scheme& s = sch();
  auto& set = for_lt ? s.lt_keys : s.rot_keys;
  REQUIRE(set.count(galel), std::string("missing Galois key for element ") + std::to_string(galel));
  return s.gkeys.at(galel)->p;
}

// ============================================================================
// key generation (GPU), identical specification to the checker
// ============================================================================
void gen_secret() {
  Scheme& s = sch();
  const int N = s.N, nm = s.L + s.K;
  s.s = ternary_hw(s.seed, ST_SK, N, s.h);
  DevArray<int8_t> ds(N); upload(ds.p, s.s.data(), N);
  s.sR = DU64((size_t)nm * N);
  launch_signed_rows(s.sR.p, rows_all(), ds.p, s.d_mods.p, N, s.st);
  ntt(s.sR.p, 0, 1, rows_all(), true);
  launch_mont_convert(s.sR.p, 0, 1, rows_all(), s.d_mods.p, N, true, s.st);
  sync();
  s.has_sk = true;
}
void gen_public() {
  Scheme& s = sch();
  REQUIRE(s.has_sk, "secret key not generated");
  const int N = s.N, nm = s.L + s.K;
  DU64 b((size_t)nm * N), a((size_t)nm * N);
  launch_sample_uniform(a.p, rows_all(), s.seed, ST_PK_A, s.d_mods.p, N, s.st);
  ntt(a.p, 0, 1, rows_all(), true);
  launch_sample_cbd(b.p, rows_all(), s.seed, ST_PK_E, s.d_mods.p, N, false, s.st);
  ntt(b.p, 0, 1, rows_all(), true);
  launch_gk_combine(b.p, a.p, s.sR.p, s.sR.p, 0, 0, s.pmod_plain.p, nm, s.d_mods.p, N, s.st);
  s.pkR = DU64((size_t)2 * nm * N);
  d2d(s.pkR.p, b.p, (size_t)nm * N * 8);
  d2d(s.pkR.p + (size_t)nm * N, a.p, (size_t)nm * N * 8);
  launch_mont_convert(s.pkR.p, (size_t)nm * N, 2, rows_all(), s.d_mods.p, N, true, s.st);
  sync();
  s.has_pk = true;
}
// Evaluation key from s_in to s_out (NTT, Montgomery form, all QP rows):
// dnum digits of (b_d, a_d), b_d = -a_d s_out + e_d + [P s_in on the rows of digit d].
template <class FA, class FE>
std::unique_ptr<DU64> gen_eval_key(const u64* s_inR, const u64* s_outR, FA st_a, FE st_e) {
  Scheme& s = sch();
  const int N = s.N, nm = s.L + s.K, K = s.K;
  auto key = std::make_unique<DU64>((size_t)s.dnum * 2 * nm * N);
  for (int d = 0; d < s.dnum; d++) {
    u64* b = key->p + (size_t)d * 2 * nm * N;
    u64* a = b + (size_t)nm * N;
    // a is sampled uniformly in the NTT domain (a uniform polynomial is
    // uniform in either domain; Lattigo's key generator samples it there too),
    // so any word of it is a function of (seed, stream, modulus, position)
    launch_sample_uniform(a, rows_all(), s.seed, st_a(d), s.d_mods.p, N, s.st);
    launch_sample_cbd(b, rows_all(), s.seed, st_e(d), s.d_mods.p, N, false, s.st);
    ntt(b, 0, 1, rows_all(), true);
    launch_gk_combine(b, a, s_outR, s_inR, d * K, std::min((d + 1) * K, s.L), s.pmod_plain.p, nm, s.d_mods.p, N, s.st);
  }
  launch_mont_convert(key->p, (size_t)nm * N, 2 * s.dnum, rows_all(), s.d_mods.p, N, true, s.st);
  sync();
  return key;
}
void ensure_galois_key(u64 galel) {
  Scheme& s = sch();
  if (s.gkeys.count(galel)) return;
  REQUIRE(s.has_sk, "secret key not generated");
  // the key-product kernels sum at most 16 digit products per accumulator
  REQUIRE(s.dnum <= 16, "key switching needs at most 16 decomposition digits (len(Q) <= 16 * len(P))");
  const int N = s.N, nm = s.L + s.K;
  u64 M = 2 * (u64)N, ginv = invmod_odd(galel, M);
  std::vector<int8_t> so(N, 0);
  for (int i = 0; i < N; i++) { u64 t = ((u64)i * ginv) % M; if (t < (u64)N) so[t] = (int8_t)(so[t] + s.s[i]); else so[t - N] = (int8_t)(so[t - N] - s.s[i]); }
  DevArray<int8_t> dso(N); upload(dso.p, so.data(), N);
  DU64 soR((size_t)nm * N);
  launch_signed_rows(soR.p, rows_all(), dso.p, s.d_mods.p, N, s.st);
  ntt(soR.p, 0, 1, rows_all(), true);
  launch_mont_convert(soR.p, 0, 1, rows_all(), s.d_mods.p, N, true, s.st);
  s.gkeys[galel] = gen_eval_key(s.sR.p, soR.p, [galel](int d) { return ST_GK_A(galel, (u64)d); },
                                 [galel](int d) { return ST_GK_E(galel, (u64)d); });
  s.seeded_gk.insert(galel);
  perm_for(galel); perm_inv_for(galel);
  // transforms cache key addresses: a key created after a removal lives elsewhere
  for (auto& kv : s.lts) kv.second->ptrs_ready = false;
}
// Relinearization key: s^2 -> s (Lattigo GenRelinearizationKey), same
// generator as the oracle's, random streams ST_RLK_A/E(d).
void ensure_relin_key() {
  Scheme& s = sch();
  if (s.rlk) return;
  REQUIRE(s.has_sk, "secret key not generated");
  REQUIRE(s.dnum <= 16, "key switching needs at most 16 decomposition digits (len(Q) <= 16 * len(P))");
  const int N = s.N, nm = s.L + s.K;
  DU64 s2R((size_t)nm * N);  // s^2 in Montgomery form: mont_mul(sR, sR) = s^2 R
  launch_mont_mul(s2R.p, 0, s.sR.p, 0, s.sR.p, 0, 1, rows_all(), s.d_mods.p, N, false, s.st);
  s.rlk = gen_eval_key(s2R.p, s.sR.p, [](int d) { return ST_RLK_A((u64)d); }, [](int d) { return ST_RLK_E((u64)d); });
  s.rlk_seeded = true;
}
// rand64's per-stream key: the kernels regenerate word (m, x) of a key's a
// half of digit d as floor(mix64(kd ^ (ctr*M1 + M2)) * q / 2^64), ctr = m*N + x
u64 stream_key(u64 stream) { return mix64(sch().seed + 0x9e3779b97f4a7c15ULL * (stream + 1)); }


// ============================================================================
// encoder: root and rotation-group tables (Lattigo ckks.Encoder); the special
// inverse FFT, fixed-point rounding and residues run on the GPU (encoder.hip),
// the decoder's forward special FFT on the host
// ============================================================================
void init_encoder(Scheme& s) {
  const int M = 2 * s.N, slots = s.N / 2, quarm = M >> 2;
  s.rre.assign(M + 1, 0.0); s.rim.assign(M + 1, 0.0);
  const double angle = 2.0 * 3.141592653589793 / (double)M;
  for (int i = 0; i < quarm; i++) s.rre[i] = std::cos(angle * (double)i);
  for (int i = 0; i < quarm; i++) s.rim[quarm - i] += s.rre[i];
  for (int i = 1; i < quarm + 1; i++) { s.rre[i + quarm] = -s.rre[quarm - i]; s.rim[i + quarm] = s.rim[quarm - i]; }
  for (int i = 1; i < quarm + 1; i++) { s.rre[i + 2 * quarm] = -s.rre[i]; s.rim[i + 2 * quarm] = -s.rim[i]; }
  for (int i = 1; i < quarm; i++) { s.rre[i + 3 * quarm] = s.rre[quarm - i]; s.rim[i + 3 * quarm] = -s.rim[quarm - i]; }
  s.rre[M] = s.rre[0]; s.rim[M] = s.rim[0];
  s.rotgroup.resize(slots);
  u64 p = 1;
  for (int j = 0; j < slots; j++) { s.rotgroup[j] = (int)p; p = (p * 5) & (u64)(M - 1); }
  s.d_rre = DevArray<double>(s.rre.size()); upload(s.d_rre.p, s.rre.data(), s.rre.size());
  s.d_rim = DevArray<double>(s.rim.size()); upload(s.d_rim.p, s.rim.data(), s.rim.size());
  s.d_rotgroup = DevArray<int>(slots); upload(s.d_rotgroup.p, s.rotgroup.data(), slots);
}
void bitrev(std::vector<double>& re, std::vector<double>& im, int n) {
  int logn = 0; while ((1 << logn) < n) logn++;
  for (int i = 0; i < n; i++) { int j = brv(i, logn); if (j > i) { std::swap(re[i], re[j]); std::swap(im[i], im[j]); } }
}
void special_fft(const Scheme& s, std::vector<double>& re, std::vector<double>& im, int n) {
  const int M = 2 * s.N;
  bitrev(re, im, n);
  for (int len = 2; len <= n; len <<= 1) {
    int lenh = len >> 1, lenq = len << 2, gap = M / lenq, mask = lenq - 1;
    for (int i = 0; i < n; i += len)
      for (int j = 0; j < lenh; j++) {
        int k = i + j;
        int idx = (s.rotgroup[j] & mask) * gap;
        double wr = s.rre[idx], wi = s.rim[idx];
        double ur = re[k], ui = im[k], xr = re[k + lenh], xi = im[k + lenh];
        double vr = xr * wr - xi * wi, vi = xr * wi + xi * wr;
        re[k] = ur + vr; im[k] = ui + vi;
        re[k + lenh] = ur - vr; im[k + lenh] = ui - vi;
      }
  }
}
// Encode np plaintexts on the device: plaintext p reads data[src[p].src * slots
// + ((k + src[p].rot) mod slots)] (zero past nvals), its residues go to rows
// rm of out + p * out_pstride, then the forward NTT.  Batches of up to 64
// plaintexts share one work buffer.
// chunk_done: nullptr -> the np plaintexts go to out (out_pstride apart);
// else out holds one chunk of up to 64 plaintexts, handed to chunk_done(c0, n)
// after each chunk is encoded (before the next overwrites it)
void encode_device(const float* h_data, size_t ndata, const std::vector<EncodeSrc>& src, int nvals, double scale, RowMap rm,
                   u64* out, size_t out_pstride, bool complex_in = false,
                   const std::function<void(int, int)>& chunk_done = nullptr) {
  Scheme& s = sch();
  const int N = s.N, slots = N / 2;
  DevArray<float> dd(std::max<size_t>(ndata, 1));
  if (ndata) upload(dd.p, h_data, ndata);
  const int np = (int)src.size(), chunk = std::min(np, 64);
  DevArray<EncodeSrc> ds(np); upload(ds.p, src.data(), np);
  DevArray<double> re((size_t)chunk * slots), im((size_t)chunk * slots);
  for (int c0 = 0; c0 < np; c0 += chunk) {
    const int nb = std::min(chunk, np - c0);
    u64* o = chunk_done ? out : out + (size_t)c0 * out_pstride;
    launch_encode_fft(o, out_pstride, rm, dd.p, ds.p + c0, nb, nvals, scale, re.p, im.p, slots, s.d_rotgroup.p, s.d_rre.p,
                      s.d_rim.p, s.d_mods.p, s.logN, s.st, complex_in);
    ntt(o, out_pstride, nb, rm, true);
    if (chunk_done) chunk_done(c0, nb);
  }
  sync();
}

// ---- big integers for the decoder's centred CRT ----
struct Big { std::vector<u64> w; };
void big_norm(Big& a) { while (!a.w.empty() && a.w.back() == 0) a.w.pop_back(); }
void big_mul_small(Big& a, u64 m) {
  u128 c = 0;
  for (auto& x : a.w) { u128 t = (u128)x * m + c; x = (u64)t; c = t >> 64; }
  if (c) a.w.push_back((u64)c);
  big_norm(a);
}
int big_cmp(const Big& a, const Big& b) {
  if (a.w.size() != b.w.size()) return a.w.size() < b.w.size() ? -1 : 1;
  for (size_t i = a.w.size(); i-- > 0;) if (a.w[i] != b.w[i]) return a.w[i] < b.w[i] ? -1 : 1;
  return 0;
}
void big_add(Big& a, const Big& b) {
  size_t n = std::max(a.w.size(), b.w.size()); a.w.resize(n, 0); u64 c = 0;
  for (size_t i = 0; i < n; i++) { u128 t = (u128)a.w[i] + (i < b.w.size() ? b.w[i] : 0) + c; a.w[i] = (u64)t; c = (u64)(t >> 64); }
  if (c) a.w.push_back(c);
}
void big_sub(Big& a, const Big& b) {  // a >= b
  u64 br = 0;
  for (size_t i = 0; i < a.w.size(); i++) { u128 t = (u128)a.w[i] - (i < b.w.size() ? b.w[i] : 0) - br; a.w[i] = (u64)t; br = (u64)(t >> 64) ? 1 : 0; }
  big_norm(a);
}
double big_to_double(const Big& a) {  // nearest, ties to even
  if (a.w.empty()) return 0.0;
  int top = (int)a.w.size() - 1, lz = __builtin_clzll(a.w[top]);
  int bitlen = top * 64 + (64 - lz);
  if (bitlen <= 64) return (double)a.w[0];
  int sh = bitlen - 64, wi = sh / 64, bi = sh % 64;
  u64 hi = bi ? (a.w[wi] >> bi) | (a.w[wi + 1] << (64 - bi)) : a.w[wi];
  bool sticky = bi && (a.w[wi] & ((1ULL << bi) - 1));
  for (int i = 0; i < wi; i++) if (a.w[i]) sticky = true;
  if (sticky) hi |= 1;
  return std::ldexp((double)hi, sh);
}
// Lattigo Encoder.Decode (float64): centred CRT value / scale, SpecialFFT, real part
std::vector<double> decode_host(const std::vector<u64>& coef, int level, double scale, std::vector<double>* imag = nullptr) {
  Scheme& s = sch();
  const int N = s.N, slots = N / 2, nl = level + 1;
  std::vector<double> vals(N);
  if (level == 0) {
    u64 q = s.mod[0];
    for (int x = 0; x < N; x++) { u64 v = coef[x]; vals[x] = (v >= (q >> 1) ? -(double)(q - v) : (double)v) / scale; }
  } else {
    Big Q; Q.w = {1};
    for (int i = 0; i < nl; i++) big_mul_small(Q, s.mod[i]);
    Big Qh = Q;
    for (size_t i = 0; i < Qh.w.size(); i++) Qh.w[i] = (Qh.w[i] >> 1) | (i + 1 < Qh.w.size() ? Qh.w[i + 1] << 63 : 0);
    big_norm(Qh);
    std::vector<Big> hat(nl); std::vector<u64> hinv(nl);
    for (int i = 0; i < nl; i++) {
      hat[i].w = {1}; u64 pr = 1;
      for (int j = 0; j < nl; j++) if (j != i) { big_mul_small(hat[i], s.mod[j]); pr = mulmod(pr, s.mod[j] % s.mod[i], s.mod[i]); }
      hinv[i] = invmod(pr, s.mod[i]);
    }
    auto work = [&](int x0, int x1) {
      for (int x = x0; x < x1; x++) {
        Big acc;
        for (int i = 0; i < nl; i++) {
          u64 y = mulmod(coef[(size_t)i * N + x], hinv[i], s.mod[i]);
          Big t = hat[i]; big_mul_small(t, y); big_add(acc, t);
        }
        while (big_cmp(acc, Q) >= 0) big_sub(acc, Q);
        double d;
        if (big_cmp(acc, Qh) >= 0) { Big t = Q; big_sub(t, acc); d = -big_to_double(t); }
        else d = big_to_double(acc);
        vals[x] = d / scale;
      }
    };
    int nt = (int)std::min<unsigned>(16, std::max(1u, std::thread::hardware_concurrency()));
    if (N < 4096) nt = 1;
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++) th.emplace_back(work, (int)((long)N * t / nt), (int)((long)N * (t + 1) / nt));
    for (auto& t : th) t.join();
  }
  std::vector<double> re(slots), im(slots);
  for (int i = 0; i < slots; i++) { re[i] = vals[i]; im[i] = vals[i + slots]; }
  special_fft(s, re, im, slots);
  if (imag) *imag = im;
  return re;
}

// ============================================================================
// scheme construction
// ============================================================================
void build_scheme(int logN, const std::vector<u64>& q, const std::vector<u64>& p, int logscale, int h, u64 seed) {
  REQUIRE(logN >= 10 && logN <= 16, "LogN must be in [10, 16] on this backend");
  REQUIRE(!q.empty() && !p.empty(), "need at least one Q and one P prime");
  REQUIRE(q.size() + p.size() <= HCK_MAXMOD, "too many moduli");
  if (!g_pool) g_pool = new Pool();
  auto sp = std::make_unique<Scheme>();
  Scheme& s = *sp;
  s.logN = logN; s.N = 1 << logN; s.L = (int)q.size(); s.K = (int)p.size();
  s.dnum = (s.L + s.K - 1) / s.K; s.logscale = logscale; s.h = h; s.seed = seed;
  REQUIRE(s.K <= HCK_MAXSRC, "too many special primes");
  s.mod = q; s.mod.insert(s.mod.end(), p.begin(), p.end());
  for (u64 m : s.mod) {
    REQUIRE(m < (1ULL << 61) && m > 2, "moduli must be < 2^61");
    REQUIRE((m - 1) % (2 * (u64)s.N) == 0, "moduli must be 1 mod 2N");
    REQUIRE(is_prime(m), "moduli must be prime");
  }
  for (size_t i = 0; i < s.mod.size(); i++) for (size_t j = i + 1; j < s.mod.size(); j++) REQUIRE(s.mod[i] != s.mod[j], "moduli must be distinct");
  HCHECK(hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking));
  s.streams[0] = s.st;
  if (g_pool) g_pool->cur = 0;
  Scheme* old = S; S = sp.get();
  try {
    const int N = s.N, nm = s.L + s.K;
    s.hmods.resize(nm);
    for (int m = 0; m < nm; m++) {
      u64 qq = s.mod[m];
      u64 inv = 1; for (int it = 0; it < 7; it++) inv *= 2 - qq * inv;  // q^-1 mod 2^64
      u64 rmod = (u64)(((u128)1 << 64) % qq);
      s.hmods[m] = ModC{qq, (u64)0 - inv, mulmod(rmod, rmod, qq), rmod};
    }
    s.d_mods = DevArray<ModC>(nm); upload(s.d_mods.p, s.hmods.data(), nm);
    std::vector<u64> htw((size_t)nm * N * 2), hitw((size_t)nm * N * 2), hn(nm), hnp(nm);
    std::vector<u64> hiu(nm), hiup(nm), hniu(nm), hniup(nm);
    std::vector<FpC> hfpc(nm, FpC{});
    for (int m = 0; m < nm; m++) {
      u64 qq = s.mod[m];
      u64 g = smallest_generator(qq);
      u64 psi = powmod(g, (qq - 1) / (2 * (u64)N), qq), ipsi = invmod(psi, qq);
      std::vector<u64> pw(N), ipw(N);
      pw[0] = ipw[0] = 1;
      for (int i = 1; i < N; i++) { pw[i] = mulmod(pw[i - 1], psi, qq); ipw[i] = mulmod(ipw[i - 1], ipsi, qq); }
      for (int i = 0; i < N; i++) {
        int r = brv(i, logN);
        const size_t o = ((size_t)m * N + i) * 2;
        htw[o] = pw[r]; htw[o + 1] = shoup(pw[r], qq);
        hitw[o] = ipw[r]; hitw[o + 1] = shoup(ipw[r], qq);
      }
      hn[m] = invmod((u64)N, qq); hnp[m] = shoup(hn[m], qq);
      hiu[m] = pw[N / 2]; hiup[m] = shoup(hiu[m], qq);
      hniu[m] = qq - pw[N / 2]; hniup[m] = shoup(hniu[m], qq);
      if (qq <= FP_QMAX) {
        // float64 transform: (w, fl(w / q)) with w centred in (-q/2, q/2]
        const double qd = (double)qq;
        auto cen = [&](u64 w) { return w > qq / 2 ? (double)w - qd : (double)w; };
        auto bits = [](double x) { u64 b; std::memcpy(&b, &x, 8); return b; };
        for (size_t k = 0; k < (size_t)N; k++) {
          const size_t o = ((size_t)m * N + k) * 2;
          const double w = cen(htw[o]), iw = cen(hitw[o]);
          htw[o] = bits(w); htw[o + 1] = bits(w / qd);
          hitw[o] = bits(iw); hitw[o + 1] = bits(iw / qd);
        }
        const double ni = cen(hn[m]), wn = cen(mulmod(ipw[brv(1, logN)], hn[m], qq));
        hfpc[m] = FpC{qd, 1.0 / qd, 4503599627370496.0 + qd, ni, ni / qd, wn, wn / qd, 0.0};
      }
    }
    auto up = [&](DU64& d, const std::vector<u64>& h) { d = DU64(h.size()); upload(d.p, h.data(), h.size()); };
    up(s.iu, hiu); up(s.iup, hiup); up(s.niu, hniu); up(s.niup, hniup);
    // lane-interleaved copies of the twiddles of the row pass's round over 16
    // consecutive words: [mod][R][slot][lane], slots in the kernel's order
    int SA, SB;
    ntt_split(logN, &SA, &SB);
    const int C = 1 << SB, R = 1 << SA, PB = 1 << (SB - 4), NST = SB - 4, NSL = ntt_row_round_slots(logN);
    std::vector<u64> htwr((size_t)nm * R * NSL * PB * 2), hitwr(htwr.size());
    for (int m = 0; m < nm; m++)
      for (int r = 0; r < R; r++)
        for (int j = 0; j < PB; j++) {
          const u64 A = (u64)r * C + 16 * (u64)j;
          for (int dir = 0; dir < 2; dir++) {
            const std::vector<u64>& src = dir == 0 ? htw : hitw;
            std::vector<u64>& dst = dir == 0 ? htwr : hitwr;
            int sl = 0;
            for (int st = 0; st < NST; st++) {
              const int lrd = dir == 0 ? NST - 1 - st : st, sh = lrd + 1;
              const u64 tb = ((u64)N + A) >> sh;
              for (int k = 0; k < (16 >> sh); k++, sl++) {
                const size_t o = ((((size_t)m * R + r) * NSL + sl) * PB + j) * 2, si = ((size_t)m * N + tb + k) * 2;
                dst[o] = src[si];
                dst[o + 1] = src[si + 1];
              }
            }
          }
        }
    up(s.tw2, htw); up(s.itw2, hitw); up(s.twr2, htwr); up(s.itwr2, hitwr); up(s.ninv, hn); up(s.ninvp, hnp);
    s.fpc = DevArray<FpC>(nm); upload(s.fpc.p, hfpc.data(), nm);
    s.tw = NttTables{s.d_mods.p, s.tw2.p, s.itw2.p, s.twr2.p, s.itwr2.p, s.ninv.p, s.ninvp.p, s.fpc.p};
    std::vector<u64> pm(nm), pmp(nm), pin(nm), pinp(nm), p0i(nm), p0ip(nm), pmr(nm);
    for (int m = 0; m < nm; m++) {
      u64 qq = s.mod[m], P = 1;
      for (int j = 0; j < s.K; j++) P = mulmod(P, s.mod[s.L + j] % qq, qq);
      pm[m] = P; pmp[m] = shoup(P, qq);
      pmr[m] = P;  // P mod q, multiplied against s*R by the Galois-key kernel
      pin[m] = m < s.L ? invmod(P, qq) : 0; pinp[m] = shoup(pin[m], qq);
      p0i[m] = m < s.L ? invmod(s.mod[s.L] % qq, qq) : 0; p0ip[m] = shoup(p0i[m], qq);
    }
    up(s.pmod_w, pm); up(s.pmod_wp, pmp); up(s.pinv_w, pin); up(s.pinv_wp, pinp); up(s.p0inv_w, p0i); up(s.p0inv_wp, p0ip); up(s.pmod_plain, pmr);
    std::vector<u64> ri((size_t)s.L * s.L, 0), rip((size_t)s.L * s.L, 0);
    for (int l = 1; l < s.L; l++)
      for (int i = 0; i < l; i++) { u64 v = invmod(s.mod[l] % s.mod[i], s.mod[i]); ri[(size_t)l * s.L + i] = v; rip[(size_t)l * s.L + i] = shoup(v, s.mod[i]); }
    up(s.rs_inv, ri); up(s.rs_invp, rip);
    std::vector<u64> pri((size_t)s.L * s.L, 0), prip((size_t)s.L * s.L, 0);
    for (int l = 1; l < s.L; l++)
      for (int i = 0; i < l; i++) {
        const u64 v = mulmod(pin[i], ri[(size_t)l * s.L + i], s.mod[i]);
        pri[(size_t)l * s.L + i] = v; prip[(size_t)l * s.L + i] = shoup(v, s.mod[i]);
      }
    up(s.prs_inv, pri); up(s.prs_invp, prip);
    s.pinv_h.assign(pin.begin(), pin.end()); s.pinv_hp.assign(pinp.begin(), pinp.end());
    init_encoder(s);
    prebuild_bconv_tables();
    init_scratch();
  } catch (...) {
    S = old;
    throw;
  }
  delete old;
  sp.release();
}

// ============================================================================
// object helpers
// ============================================================================
Plain& get_pt(int id) { auto it = sch().pts.find(id); REQUIRE(it != sch().pts.end(), "plaintext not found: " + std::to_string(id)); return *it->second; }
Cipher& get_ct(int id) { auto it = sch().cts.find(id); REQUIRE(it != sch().cts.end(), "ciphertext not found: " + std::to_string(id)); return *it->second; }
LinTrans& get_lt(int id) { auto it = sch().lts.find(id); REQUIRE(it != sch().lts.end(), "linear transform not found: " + std::to_string(id)); return *it->second; }
int push_pt(std::unique_ptr<Plain> p) { Scheme& s = sch(); int id = s.pt_ids.take(); s.pts[id] = std::move(p); return id; }
int push_ct(std::unique_ptr<Cipher> c) { Scheme& s = sch(); int id = s.ct_ids.take(); s.cts[id] = std::move(c); return id; }
std::unique_ptr<Cipher> new_ct(int level, double scale) {
  Scheme& s = sch();
  auto c = std::make_unique<Cipher>();
  c->level = level; c->scale = scale; c->logslots = s.logN - 1;
  c->d = DU64((size_t)2 * (level + 1) * s.N);
  return c;
}
std::unique_ptr<Cipher> copy_ct(const Cipher& a) {
  auto c = new_ct(a.level, a.scale); c->logslots = a.logslots;
  d2d(c->d.p, a.d.p, a.d.bytes());
  return c;
}
// drop ciphertext limbs above `level`
void ct_drop_to(Cipher& c, int level) {
  Scheme& s = sch();
  if (c.level == level) return;
  DU64 d((size_t)2 * (level + 1) * s.N);
  copy_rows(d.p, (size_t)(level + 1) * s.N, c.d.p, (size_t)(c.level + 1) * s.N, (size_t)(level + 1) * s.N, 2);
  c.d = std::move(d); c.level = level;
}

// ============================================================================
// evaluator operations
// ============================================================================
// Key-switched automorphism of ct into out (2 (l+1) N words, out != ct):
// c1 decomposed and extended to QP, key product fused with nothing else,
// ModDown of both parts with sigma applied in its epilogue and c0 added.
// ws: nullptr -> temporaries from the buffer cache; else
// automorphism_ws_words(l) device words laid out as
//   [digits (dn nqp N), later ModDown's pc and ext | dd (2 nqp N) | coef ((l+1) N)]
// (the digits are dead once the key product has read them).
size_t automorphism_ws_words(int l) {
  Scheme& s = sch();
  const size_t N = s.N, K = s.K, nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
  return (std::max(dn * nqp, 2 * K + 2 * (size_t)(l + 1)) + 2 * nqp + (size_t)(l + 1)) * N;
}
// acc: nullptr, or a ciphertext at ct's level (not out) added to the result
void automorphism_core(const Cipher& ct, u64 galel, const u64* key, const uint32_t* perm_inv, u64* out, u64* ws,
                       const u64* acc = nullptr) {
  Scheme& s = sch();
  const int l = ct.level, N = s.N, K = s.K, nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
  DU64 digits_buf, dd_buf;
  u64 *digits, *dd, *coef = nullptr, *md = nullptr;
  if (ws) {
    digits = ws;
    md = ws;
    dd = ws + std::max((size_t)dn * nqp, 2 * (size_t)K + 2 * (size_t)(l + 1)) * N;
    coef = dd + (size_t)2 * nqp * N;
  } else {
    digits_buf = DU64((size_t)dn * nqp * N); dd_buf = DU64((size_t)2 * nqp * N);
    digits = digits_buf.p; dd = dd_buf.p;
  }
  decompose_modup(l, ct.d.p + (size_t)(l + 1) * N, 0, 1, digits, false, coef);
  KeyMacArgs a{};
  a.digits = digits; a.dig_bstride = 0; a.digits_per_batch = 0; a.key = nullptr; a.perm = nullptr;
  a.key1 = key; a.perm1 = nullptr; a.add0 = nullptr;
  a.own = ct.d.p + (size_t)(l + 1) * N; a.own_bstride = 0;
  a.out0 = dd; a.out1 = dd + (size_t)nqp * N; a.out_bstride = 0; a.mods = s.d_mods.p;
  a.N = N; a.l = l; a.L = s.L; a.K = K; a.nqp = nqp; a.dn = dn;
  if (s.seeded_gk.count(galel)) {
    a.seeded = 1;
    for (int d = 0; d < dn; d++) a.ka[d] = stream_key(ST_GK_A(galel, (u64)d));
  }
  launch_keymac(a, 1, s.st);
  mod_down(l, dd, (size_t)nqp * N, 2, out, (size_t)(l + 1) * N, ct.d.p, 0, 1, perm_inv, md, acc);
}
std::unique_ptr<Cipher> automorphism(const Cipher& ct, u64 galel, bool lt_keyset) {
  const u64* key = key_ptr(galel, lt_keyset);
  auto out = new_ct(ct.level, ct.scale); out->logslots = ct.logslots;
  timed("rotate", [&] { automorphism_core(ct, galel, key, perm_inv_for(galel), out->d.p, nullptr); });
  return out;
}
// ---- plaintext, scalar and ciphertext products (Lattigo ckks Evaluator
// Mul / Add with a constant / MulRelin, restated for the GPU) ----

// Lattigo's scaled real constant (float64 encoding precision): v * scale
// rounded to double, then +-0.5 in double, truncated toward zero.
typedef __int128 i128;
i128 scaled_constant(double v, double scale) {
  double t = v * scale;
  REQUIRE(t < 42535295865117307932921825928971026432.0 && t > -42535295865117307932921825928971026432.0,
          "scaled constant exceeds 2^125");
  if (t > 0) t = t + 0.5; else if (t < 0) t = t - 0.5;
  return (i128)t;
}
u64 residue_i64(i128 k, u64 q) {
  if (k >= 0) return (u64)((u128)k % q);
  u64 m = (u64)((u128)(-(k + 1)) % q);
  m = (m + 1) % q;
  return m ? q - m : 0;
}
// both parts of c (level l) times the integer k, in place
// (the residues travel in the kernel arguments: the host does not wait)
void mul_int_inplace(Cipher& c, i128 k) {
  Scheme& s = sch();
  const int l = c.level;
  RowConst rc{};
  for (int i = 0; i <= l; i++) { rc.w[i] = residue_i64(k, s.mod[i]); rc.wp[i] = shoup(rc.w[i], s.mod[i]); }
  launch_mul_const_v(c.d.p, c.d.p, (size_t)(l + 1) * s.N, 2, rows_q(l), rc, s.d_mods.p, s.N, s.st);
}
// Mul(ct, float64): integer-valued constants multiply as integers (scale
// unchanged); others are scaled by q_l and rounded, and the scale grows by q_l
void mul_float_inplace(Cipher& c, double v) {
  Scheme& s = sch();
  if (v < 4611686018427387904.0 && v > -4611686018427387904.0 && v == (double)(int64_t)v) {
    mul_int_inplace(c, (i128)(int64_t)v);
    return;
  }
  const i128 k = scaled_constant(v, (double)s.mod[c.level]);
  mul_int_inplace(c, k);
  c.scale *= (double)s.mod[c.level];
}
// Add(ct, float64): round(v * scale) added to (subtracted from) every NTT slot of part 0
void add_const_inplace(Cipher& c, double v, bool sub) {
  Scheme& s = sch();
  const int l = c.level;
  const i128 k = scaled_constant(v, c.scale);
  RowConst rc{};
  for (int i = 0; i <= l; i++) rc.w[i] = residue_i64(k, s.mod[i]);
  launch_add_scalar_v(c.d.p, c.d.p, rows_q(l), rc, s.d_mods.p, s.N, sub, s.st);
}
// Mul(ct, pt): both parts times the plaintext at level min(ct, pt); scales multiply
std::unique_ptr<Cipher> mul_plain_ct(const Cipher& ct, const Plain& pt) {
  Scheme& s = sch();
  const int l = std::min(ct.level, pt.level), N = s.N;
  DU64 pR((size_t)(l + 1) * N);
  d2d(pR.p, pt.d.p, (size_t)(l + 1) * N * 8);
  launch_mont_convert(pR.p, 0, 1, rows_q(l), s.d_mods.p, N, true, s.st);
  auto out = new_ct(l, ct.scale * pt.scale); out->logslots = ct.logslots;
  launch_mont_mul(out->d.p, (size_t)(l + 1) * N, ct.d.p, (size_t)(ct.level + 1) * N, pR.p, 0, 2, rows_q(l), s.d_mods.p, N,
                  false, s.st);
  return out;
}
// MulRelin(a, b): tensor (a0 b0, a0 b1 + a1 b0, a1 b1) at level min, then the
// third part key switched with the relinearization key and added.
// rescale: return Rescale(MulRelin(a, b)) (one modulus), word for word: the
// tensor's first two parts enter the key switch's Q rows multiplied by P
// (ModDown(x + P d) = ModDown(x) + d exactly: [P d]_P = 0), and the ModDown
// is fused with the rescale (mod_down_rescale), so the rescale's own inverse
// and forward transforms are not run.
std::unique_ptr<Cipher> mul_relin_ct(const Cipher& a, const Cipher& b, bool rescale) {
  Scheme& s = sch();
  REQUIRE(s.rlk, "relinearization key not generated");
  const int l = std::min(a.level, b.level), N = s.N, K = s.K, nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
  REQUIRE(!rescale || l >= 1, "cannot rescale: ciphertext already at level 0");
  const size_t ps = (size_t)(l + 1) * N;
  DU64 dt(3 * ps);
  u64 *d0 = dt.p, *d1 = dt.p + ps, *d2 = dt.p + 2 * ps;
  launch_tensor(d0, d1, d2, a.d.p, a.d.p + (size_t)(a.level + 1) * N, b.d.p, b.d.p + (size_t)(b.level + 1) * N, l,
                rescale ? s.pmod_w.p : nullptr, rescale ? s.pmod_wp.p : nullptr, s.d_mods.p, N, s.st);
  DU64 digits((size_t)dn * nqp * N), dd((size_t)2 * nqp * N);
  decompose_modup(l, d2, 0, 1, digits.p, false);
  KeyMacArgs k{};
  k.digits = digits.p; k.dig_bstride = 0; k.digits_per_batch = 0; k.key = nullptr; k.perm = nullptr;
  k.key1 = s.rlk->p; k.perm1 = nullptr;
  k.add0 = rescale ? d0 : nullptr; k.add1 = rescale ? d1 : nullptr;
  k.own = d2; k.own_bstride = 0;
  k.out0 = dd.p; k.out1 = dd.p + (size_t)nqp * N; k.out_bstride = 0; k.mods = s.d_mods.p;
  k.N = N; k.l = l; k.L = s.L; k.K = K; k.nqp = nqp; k.dn = dn;
  if (s.rlk_seeded) {
    k.seeded = 1;
    for (int d = 0; d < dn; d++) k.ka[d] = stream_key(ST_RLK_A((u64)d));
  }
  launch_keymac(k, 1, s.st);
  if (rescale) {
    auto out = new_ct(l - 1, a.scale * b.scale / (double)s.mod[l]); out->logslots = a.logslots;
    mod_down_rescale(l, dd.p, (size_t)nqp * N, 2, out->d.p, (size_t)l * N);
    return out;
  }
  auto out = new_ct(l, a.scale * b.scale); out->logslots = a.logslots;
  // out = ModDown(dd) + (d0, d1): the epilogue reads and writes each word in one thread
  mod_down(l, dd.p, (size_t)nqp * N, 2, out->d.p, ps, d0, ps, 2, nullptr);
  return out;
}
std::unique_ptr<Cipher> rescale_ct(const Cipher& ct);
void add_inplace(Cipher& a, const Cipher& b, bool sub);
// Rescale(K_g * x) + C_g (C_g added to part 0, at the output's scale) for two
// integers K_0, K_1 in one pass, word for word what mul_int_inplace,
// rescale_ct and add_const_inplace compute one after the other: the inverse
// transform of x's row l is shared (the rescale's spread takes K_g,l times
// it), and the forward transform's epilogue multiplies x by K_g,i itself.
std::pair<std::unique_ptr<Cipher>, std::unique_ptr<Cipher>> rescale_scaled_pair(const Cipher& x, i128 k0, double c0,
                                                                                 double sc0, i128 k1, double c1, double sc1) {
  Scheme& s = sch();
  const int l = x.level, N = s.N;
  REQUIRE(l >= 1, "cannot rescale: ciphertext already at level 0");
  REQUIRE(l <= HCK_MAXQ, "rescale pair: too many limbs");
  RescalePair rp{};
  const i128 ks[2] = {k0, k1};
  const double cs[2] = {c0, c1}, scs[2] = {sc0, sc1};
  for (int g = 0; g < 2; g++) {
    rp.kl[g] = residue_i64(ks[g], s.mod[l]); rp.klp[g] = shoup(rp.kl[g], s.mod[l]);
    const i128 kc = scaled_constant(cs[g], scs[g]);
    for (int i = 0; i < l; i++) {
      rp.k[g][i] = residue_i64(ks[g], s.mod[i]); rp.kp[g][i] = shoup(rp.k[g][i], s.mod[i]);
      rp.c[g][i] = residue_i64(kc, s.mod[i]);
    }
  }
  DU64 u((size_t)2 * N), t((size_t)4 * l * N), kd((size_t)6 * l);
  ntt_oop(x.d.p + (size_t)l * N, (size_t)(l + 1) * N, u.p, N, 2, RowMap{1, 1, l, 0, 0, 0}, false);
  launch_rescale_pair_spread(t.p, u.p, l, s.mod[l] >> 1, rp, kd.p, s.d_mods.p, N, s.st);
  auto a = new_ct(l - 1, x.scale / (double)s.mod[l]); a->logslots = x.logslots;
  auto b = new_ct(l - 1, x.scale / (double)s.mod[l]); b->logslots = x.logslots;
  launch_ntt_rescale_pair(t.p, (size_t)l * N, l, s.logN, x.d.p, (size_t)(l + 1) * N, a->d.p, b->d.p, (size_t)l * N, kd.p,
                          s.rs_inv.p + (size_t)l * s.L, s.rs_invp.p + (size_t)l * s.L, s.tw, s.st);
  return {std::move(a), std::move(b)};
}
// Monomial polynomial of degree <= 3 at depth ceil(log2(d + 1)), output scale
// `so` (the same composition as the restatement's orc_eval_poly):
//   d = 1: Rescale(X * K1) + c0, K1 = round(c1 * so * q_l / s)
//   d = 2, 3: X2 = Rescale(MulRelin(X, X)); B = Rescale(X * K3) + c2 at
//     scale sB = so * q_{l-1} / scale(X2), K3 = round(c3 * sB * q_l / s);
//     out = Rescale(MulRelin(X2, B)) + (Rescale(X * K1) dropped one level + c0)
std::unique_ptr<Cipher> eval_poly_ct(const Cipher& x, std::vector<double> coef, double so) {
  Scheme& s = sch();
  int d = (int)coef.size() - 1;
  while (d > 0 && coef[d] == 0.0) d--;
  REQUIRE(d >= 0 && d <= 3, "the hip backend evaluates polynomials of degree <= 3");
  const int l = x.level;
  if (d == 0) {
    auto out = copy_ct(x);
    mul_int_inplace(*out, 0);
    out->scale = so;
    add_const_inplace(*out, coef[0], false);
    return out;
  }
  REQUIRE(l >= (d == 1 ? 1 : 2), "not enough levels left for the polynomial");
  const double ql = (double)s.mod[l];
  const i128 k1 = scaled_constant(coef[1], so * ql / x.scale);
  if (d == 1) {
    auto t = copy_ct(x);
    mul_int_inplace(*t, k1);
    auto A = rescale_ct(*t);
    A->scale = so;
    add_const_inplace(*A, coef[0], false);
    return A;
  }
  const double s2 = x.scale * x.scale / ql;
  const double sB = so * (double)s.mod[l - 1] / s2;
  // A + c0 and B = Rescale(X * K3) + c2 in one rescale pass (A's rows above
  // l - 2 are not read: the final sum is at level l - 2)
  auto AB = rescale_scaled_pair(x, k1, coef[0], so, scaled_constant(d == 3 ? coef[3] : 0.0, sB * ql / x.scale), coef[2], sB);
  auto& A2 = AB.first;
  auto& B = AB.second;
  A2->scale = so;
  B->scale = sB;
  auto X2 = mul_relin_ct(x, x, true);
  X2->scale = s2;
  auto out = mul_relin_ct(*X2, *B, true);
  out->scale = so;
  add_inplace(*out, *A2, false);
  return out;
}
std::unique_ptr<Cipher> rescale_ct(const Cipher& ct) {
  Scheme& s = sch();
  const int l = ct.level, N = s.N;
  REQUIRE(l >= 1, "cannot rescale: ciphertext already at level 0");
  DU64 u((size_t)2 * N), t((size_t)2 * l * N);
  ntt_oop(ct.d.p + (size_t)l * N, (size_t)(l + 1) * N, u.p, N, 2, RowMap{1, 1, l, 0, 0, 0}, false);
  launch_rescale_spread(t.p, u.p, l, s.mod[l] >> 1, s.d_mods.p, N, s.st);
  auto out = new_ct(l - 1, ct.scale / (double)s.mod[l]); out->logslots = ct.logslots;
  // forward transform of t whose row pass ends in out_i = (x_i - t_i) * q_l^-1
  launch_ntt_moddown(t.p, (size_t)l * N, 2, l - 1, s.logN, ct.d.p, (size_t)(l + 1) * N, out->d.p, (size_t)l * N, nullptr, 0, 0,
                     nullptr, s.rs_inv.p + (size_t)l * s.L, s.rs_invp.p + (size_t)l * s.L, s.tw, s.st);
  return out;
}
// Number of moduli Lattigo's ckks Rescale divides by: the last ones, while
// the scale stays >= default/2
int lattigo_rescale_count(double scale, int level) {
  Scheme& s = sch();
  const double minscale = std::ldexp(1.0, s.logscale) / 2.0;
  double sc = scale; int lvl = level, nb = 0;
  while (lvl >= 1) { double ns = sc / (double)s.mod[lvl]; if (ns < minscale) break; sc = ns; lvl--; nb++; }
  return nb;
}
std::unique_ptr<Cipher> rescale_lattigo(const Cipher& ct) {
  REQUIRE(ct.level >= 1, "cannot rescale: ciphertext already at level 0");
  const int nb = lattigo_rescale_count(ct.scale, ct.level);
  if (nb == 0) return copy_ct(ct);
  std::unique_ptr<Cipher> cur = rescale_ct(ct);
  for (int i = 1; i < nb; i++) cur = rescale_ct(*cur);
  return cur;
}
void add_inplace(Cipher& a, const Cipher& b, bool sub) {
  Scheme& s = sch();
  REQUIRE(a.scale == b.scale, "ciphertext scales differ");
  int l = std::min(a.level, b.level);
  ct_drop_to(a, l);
  const size_t bs_b = (size_t)(b.level + 1) * s.N;
  if (b.level == l) {
    // both parts in one launch (same row stride in a and b)
    launch_add(a.d.p, a.d.p, b.d.p, bs_b, 2, rows_q(l), s.d_mods.p, s.N, sub, s.st);
    return;
  }
  for (int p = 0; p < 2; p++)
    launch_add(a.d.p + (size_t)p * (l + 1) * s.N, a.d.p + (size_t)p * (l + 1) * s.N, b.d.p + (size_t)p * bs_b, 0, 1, rows_q(l), s.d_mods.p, s.N, sub, s.st);
}
void add_plain_inplace(Cipher& a, const Plain& p, bool sub) {
  Scheme& s = sch();
  REQUIRE(a.scale == p.scale, "ciphertext and plaintext scales differ");
  int l = std::min(a.level, p.level);
  ct_drop_to(a, l);
  launch_add(a.d.p, a.d.p, p.d.p, 0, 1, rows_q(l), s.d_mods.p, s.N, sub, s.st);
}

// ============================================================================
// linear transform (lintrans restated for the GPU)
// ============================================================================
void bsgs_index(const std::vector<int>& diags, int slots, int N1, std::vector<int>& r1, std::vector<int>& r2) {
  std::set<int> a, b;
  for (int d : diags) { int r = d & (slots - 1); a.insert(((r / N1) * N1) & (slots - 1)); b.insert(r & (N1 - 1)); }
  r1.assign(a.begin(), a.end()); r2.assign(b.begin(), b.end());
}
int find_best_bsgs_ratio(const std::vector<int>& diags, int maxN, int logMaxRatio) {
  double maxRatio = (double)(1 << logMaxRatio);
  for (int N1 = 1; N1 < maxN; N1 <<= 1) {
    std::vector<int> r1, r2; bsgs_index(diags, maxN, N1, r1, r2);
    double nbN1 = (double)r1.size() - 1, nbN2 = (double)r2.size() - 1;
    double ratio = nbN2 / nbN1;
    if (ratio == maxRatio) return N1;
    if (ratio > maxRatio) return N1 / 2;
  }
  return 1;
}
std::vector<int> lt_rotations(const LinTrans& t) {
  std::vector<int> out;
  if (t.naive) { for (int r : t.rot2) out.push_back(r); return out; }
  for (int r : t.rot1) out.push_back(r);
  for (int r : t.rot2) if (std::find(out.begin(), out.end(), r) == out.end()) out.push_back(r);
  return out;
}

// The diagonal MAC reads plaintext gpi[g][b] of its diagonal buffer (np
// diagonals plus the all-zero one at index np) and the key / permutation of
// baby slot bslot[b]; every index must stay inside those arrays, and a dense
// transform (plaintext index computed as g * nbaby + b, no table) must hold
// exactly that layout.  Checked on the host before the tables are uploaded
// and again before every launch.
void check_mac_tables(const LinTrans& t) {
  const int ng = (int)t.giant.size(), nb = (int)t.rot2.size(), np = (int)t.plain_idx.size();
  REQUIRE(t.gpi.size() == (size_t)ng * nb && t.bzero.size() == (size_t)nb && t.bslot.size() == (size_t)nb,
          "linear transform: index tables do not match the baby / giant step counts");
  int nbr = 0;
  for (int b = 0; b < nb; b++) nbr += t.rot2[b] != 0;
  for (int b = 0; b < nb; b++) {
    REQUIRE(t.bzero[b] == (t.rot2[b] == 0 ? 1 : 0), "linear transform: baby-step zero flag out of step");
    REQUIRE(t.bzero[b] || (t.bslot[b] >= 0 && t.bslot[b] < nbr), "linear transform: baby-step key slot out of range");
  }
  for (size_t i = 0; i < t.gpi.size(); i++) {
    REQUIRE(t.gpi[i] >= 0 && t.gpi[i] <= np, "linear transform: plaintext index out of range");
    if (t.dense) REQUIRE(t.gpi[i] == (int)i, "linear transform: dense layout broken");
  }
}

// u64 words one stored diagonal takes
size_t lt_diag_words(const LinTrans& t) {
  Scheme& s = sch();
  return t.packed ? t.pk_stride / 2 : (size_t)(t.level + 1 + s.K) * s.N;
}
// the packed layout of a dense 16-baby transform's diagonals
void lt_pack_layout(LinTrans& t) {
  Scheme& s = sch();
  const int nqp = t.level + 1 + s.K, N = s.N;
  t.pkrow.assign((size_t)2 * nqp, 0);
  size_t off = 0;
  for (int k = 0; k < nqp; k++) {
    const u64 q = s.mod[qp_mod(t.level, k)];
    const bool pk = q < (1ull << PK_BITS) && N % 256 == 0;
    t.pkrow[2 * k] = (uint32_t)off;
    t.pkrow[2 * k + 1] = pk ? PK_BITS : 0;
    off += pk ? (size_t)(N / 64) * PK_CHUNK : (size_t)2 * N;
  }
  REQUIRE(off < (1ull << 32), "packed diagonal too large");
  t.pk_stride = off;  // every row a multiple of 4 dwords: rows and diagonals stay 16-byte aligned
  t.packed = true;
  t.d_pkrow = DevArray<uint32_t>(t.pkrow.size());
  upload(t.d_pkrow.p, t.pkrow.data(), t.pkrow.size());
}
// storage of np diagonals + the all-zero plaintext after them
void lt_alloc_diags(LinTrans& t, int np) {
  Scheme& s = sch();
  const size_t w = lt_diag_words(t);
  t.diags = DU64((size_t)(np + 1) * w);
  HCHECK(hipMemsetAsync(t.diags.p + (size_t)np * w, 0, w * 8, s.st));
}
// diagonal p of t as plain rows [nqp][N] in dst (device); store the same back
void lt_diag_get(const LinTrans& t, size_t p, u64* dst) {
  Scheme& s = sch();
  const size_t w = lt_diag_words(t);
  if (!t.packed) { d2d(dst, t.diags.p + p * w, w * 8); return; }
  launch_unpack_diag(dst, reinterpret_cast<const uint32_t*>(t.diags.p + p * w), t.d_pkrow.p, t.level + 1 + s.K, s.N, s.st);
}
void lt_diag_put(LinTrans& t, size_t p, const u64* src, int np = 1) {
  Scheme& s = sch();
  const size_t w = lt_diag_words(t), plain = (size_t)(t.level + 1 + s.K) * s.N;
  if (!t.packed) { d2d(t.diags.p + p * w, src, (size_t)np * w * 8); return; }
  launch_pack_diags(reinterpret_cast<uint32_t*>(t.diags.p + p * w), t.pk_stride, src, plain, np, t.d_pkrow.p, t.level + 1 + s.K,
                    s.N, s.st);
}

int generate_lt(const int* idx, int nidx, const float* data, int ndata, int level, float ratio, bool load_mode) {
  Scheme& s = sch();
  const int N = s.N, slots = N / 2, K = s.K;
  REQUIRE(nidx > 0, "no diagonals");
  REQUIRE(ndata == nidx * slots || (load_mode && ndata == 0), "diagonal data length must be len(diag_idxs) * slots");
  REQUIRE(level >= 0 && level < s.L, "invalid level");
  auto t = std::make_unique<LinTrans>();
  t->level = level; t->slots = slots;
  t->keys.assign(idx, idx + nidx);
  int logratio = (int)std::log((double)ratio);
  t->scale = (double)s.mod[level];
  std::vector<std::pair<int, int>> order;  // (diag index, source row)
  auto src_of = [&](int di) { for (int i = 0; i < nidx; i++) if (idx[i] == di || idx[i] == di - slots) return i; throw Error("lintrans: diagonal missing"); };
  std::vector<int> rotv;  // pre-rotation per plaintext
  if (logratio < 0) {
    t->naive = true; t->N1 = 0;
    bsgs_index(t->keys, slots, slots, t->rot1, t->rot2);
    for (int i = 0; i < nidx; i++) { int di = idx[i] < 0 ? idx[i] + slots : idx[i]; order.push_back({di, i}); rotv.push_back(0); }
  } else {
    t->N1 = find_best_bsgs_ratio(t->keys, slots, logratio);
    REQUIRE(t->N1 >= 1, "invalid baby-step size");
    bsgs_index(t->keys, slots, t->N1, t->rot1, t->rot2);
    t->giant = t->rot1;
    t->baby.assign(t->giant.size(), {});
    for (int d : t->keys) {
      int r = d & (slots - 1), j = ((r / t->N1) * t->N1) & (slots - 1), b = r & (t->N1 - 1);
      size_t g = std::lower_bound(t->giant.begin(), t->giant.end(), j) - t->giant.begin();
      t->baby[g].push_back(b);
    }
    for (auto& bl : t->baby) { std::sort(bl.begin(), bl.end()); bl.erase(std::unique(bl.begin(), bl.end()), bl.end()); }
    for (size_t g = 0; g < t->giant.size(); g++)
      for (int b : t->baby[g]) { int di = t->giant[g] + b; order.push_back({di, src_of(di)}); rotv.push_back((-t->giant[g]) & (slots - 1)); }
  }
  const int np = (int)order.size(), nqp_lt = level + 1 + K;
  for (auto& o : order) t->plain_idx.push_back(o.first);
  if (!t->naive) {
    const int ng = (int)t->giant.size(), nb = (int)t->rot2.size();
    std::vector<int> gpi((size_t)ng * nb, np), bzero(nb, 0), bslot(nb, 0);
    int pidx = 0;
    for (int g = 0; g < ng; g++)
      for (int b : t->baby[g]) {
        int pos = (int)(std::lower_bound(t->rot2.begin(), t->rot2.end(), b) - t->rot2.begin());
        gpi[(size_t)g * nb + pos] = pidx++;
      }
    t->dense = true;
    for (size_t i = 0; i < gpi.size(); i++) if (gpi[i] != (int)i) t->dense = false;
    int slot = 0;
    for (int i = 0; i < nb; i++) { bzero[i] = t->rot2[i] == 0; bslot[i] = t->rot2[i] == 0 ? 0 : slot++; }
    t->gpi = std::move(gpi); t->bzero = std::move(bzero); t->bslot = std::move(bslot);
    check_mac_tables(*t);
    t->d_gpi = DevArray<int>(t->gpi.size()); upload(t->d_gpi.p, t->gpi.data(), t->gpi.size());
    t->d_bzero = DevArray<int>(nb); upload(t->d_bzero.p, t->bzero.data(), nb);
    t->d_bslot = DevArray<int>(nb); upload(t->d_bslot.p, t->bslot.data(), nb);
    // the diagonal MAC's dense 16-baby kernel reads packed diagonals
    if (t->dense && nb == 16) lt_pack_layout(*t);
  }
  if (load_mode) {
    // io_mode "load" (lineartransform.go:75-84): empty diagonal slots, filled by LoadPlaintextDiagonal
    t->resident.assign(np, 0);
  } else {
    // one extra all-zero plaintext after the np diagonals: absent (group, baby) pairs point at it
    lt_alloc_diags(*t, np);
    RowMap rm{nqp_lt, level + 1, 0, s.L, 0, 0};
    // special FFT, fixed point, residues in QP and NTT on the device, then the
    // Montgomery conversion; packed transforms encode through a plain staging
    // buffer of up to 64 diagonals at a time
    const size_t plain = (size_t)nqp_lt * N;
    std::vector<EncodeSrc> src(np);
    for (int p = 0; p < np; p++) src[p] = EncodeSrc{order[p].second, rotv[p]};
    if (!t->packed) {
      encode_device(data, (size_t)ndata, src, slots, t->scale, rm, t->diags.p, plain);
      launch_mont_convert(t->diags.p, plain, np, rm, s.d_mods.p, N, true, s.st);
    } else {
      DU64 stage((size_t)std::min(np, 64) * plain);
      encode_device(data, (size_t)ndata, src, slots, t->scale, rm, stage.p, plain, false, [&](int c0, int n) {
        launch_mont_convert(stage.p, plain, n, rm, s.d_mods.p, N, true, s.st);
        lt_diag_put(*t, (size_t)c0, stage.p, n);
      });
    }
    t->resident.assign(np, 1);
  }
  sync();
  int id = s.lt_ids.take();
  s.lts[id] = std::move(t);
  return id;
}

// MultiplyByDiagMatrixBSGS on the GPU: one decomposition, one fused pass that
// computes the hoisted baby rotations and the diagonal MAC producing every
// giant group's QP accumulators, batched ModDown + decomposition of the giant groups' c1
// parts, one fused key-product/automorphism/accumulate pass, final ModDown.
// rescale: return Rescale(result) (Lattigo's ckks Rescale), with the first
// division fused into the final ModDown
std::unique_ptr<Cipher> eval_lt_bsgs(const LinTrans& t, const Cipher& ct, bool rescale) {
  Scheme& s = sch();
  const int N = s.N, K = s.K;
  const int l = std::min(ct.level, t.level), nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
  const size_t qp = (size_t)nqp * N;
  const u64* c0 = ct.d.p;
  const u64* c1 = ct.d.p + (size_t)(ct.level + 1) * N;
  // 1. decomposition of c1 and P*c
  DU64 digits((size_t)dn * qp);
  decompose_modup(l, c1, 0, 1, digits.p, false);
  DU64 pc((size_t)2 * (l + 1) * N);
  launch_mul_const(pc.p, c0, 0, 1, rows_q(l), s.pmod_w.p, s.pmod_wp.p, s.d_mods.p, N, s.st);
  launch_mul_const(pc.p + (size_t)(l + 1) * N, c1, 0, 1, rows_q(l), s.pmod_w.p, s.pmod_wp.p, s.d_mods.p, N, s.st);
  std::vector<int> babies;
  for (int b : t.rot2) if (b != 0) babies.push_back(b);
  const int nbr = (int)babies.size();
  const int ng = (int)t.giant.size(), nb = (int)t.rot2.size();
  const int gs = (ng > 0 && t.giant[0] == 0) ? 1 : 0;
  const int ngk = ng - gs;
  {
    // every key must be in the transform key set (checked on each call); pointer tables are uploaded once
    std::vector<const u64*> bk(nbr), gk(ngk); std::vector<const uint32_t*> bp(nbr), gp(ngk); std::vector<int> tg(ngk);
    for (int i = 0; i < nbr; i++) { u64 ge = galois_element(babies[i]); bk[i] = key_ptr(ge, true); bp[i] = perm_for(ge); }
    for (int g = 0; g < ngk; g++) { u64 ge = galois_element(t.giant[gs + g]); gk[g] = key_ptr(ge, true); gp[g] = perm_for(ge); tg[g] = gs + g; }
    LinTrans& tm = const_cast<LinTrans&>(t);
    if (!tm.ptrs_ready) {
      tm.d_bkey = DevArray<const u64*>(std::max(nbr, 1)); tm.d_bperm = DevArray<const uint32_t*>(std::max(nbr, 1));
      tm.d_gkey = DevArray<const u64*>(std::max(ngk, 1)); tm.d_gperm = DevArray<const uint32_t*>(std::max(ngk, 1));
      tm.d_tg = DevArray<int>(std::max(ngk, 1));
      if (nbr) { upload(tm.d_bkey.p, bk.data(), nbr); upload(tm.d_bperm.p, bp.data(), nbr); }
      if (ngk) { upload(tm.d_gkey.p, gk.data(), ngk); upload(tm.d_gperm.p, gp.data(), ngk); upload(tm.d_tg.p, tg.data(), ngk); }
      // the stream keys depend on the Galois element alone
      std::vector<u64> bka((size_t)std::max(nbr, 1) * dn), gka((size_t)std::max(ngk, 1) * dn);
      for (int i = 0; i < nbr; i++)
        for (int d = 0; d < dn; d++) bka[(size_t)i * dn + d] = stream_key(ST_GK_A(galois_element(babies[i]), (u64)d));
      for (int g = 0; g < ngk; g++)
        for (int d = 0; d < dn; d++) gka[(size_t)g * dn + d] = stream_key(ST_GK_A(galois_element(t.giant[gs + g]), (u64)d));
      tm.d_bka = DevArray<u64>(bka.size()); upload(tm.d_bka.p, bka.data(), bka.size());
      tm.d_gka = DevArray<u64>(gka.size()); upload(tm.d_gka.p, gka.data(), gka.size());
      tm.ptrs_ready = true;
    }
  }
  // the a halves are regenerated in the kernels when every key of the group
  // of launches was generated here (a loaded key is read whole)
  bool babies_seeded = true, giants_seeded = true;
  for (int i = 0; i < nbr; i++) babies_seeded = babies_seeded && s.seeded_gk.count(galois_element(babies[i]));
  for (int g = 0; g < ngk; g++) giants_seeded = giants_seeded && s.seeded_gk.count(galois_element(t.giant[gs + g]));
  // 2. the hoisted baby rotations (sigma(d0 + P c0), sigma(d1)) are computed by
  // the diagonal MAC in its prologue (keymac_kernel's arithmetic per word), so
  // they never go through memory
  // 3. fused diagonal MAC -> T[g][2][nqp][N]
  DU64 T((size_t)ng * 2 * qp);
  DiagMacArgs dm{};
  dm.diag = t.diags.p; dm.diag_stride = lt_diag_words(t);
  dm.pkrow = t.packed ? t.d_pkrow.p : nullptr;
  dm.digits = digits.p; dm.bkey = t.d_bkey.p; dm.bperm = t.d_bperm.p; dm.own = c1; dm.dn = dn;
  dm.bka = babies_seeded ? t.d_bka.p : nullptr;
  dm.pc = pc.p; dm.pc_pstride = (size_t)(l + 1) * N;
  dm.baby_is_zero = t.d_bzero.p; dm.baby_slot = t.d_bslot.p; dm.gpi = t.d_gpi.p; dm.dense = t.dense ? 1 : 0;
  dm.zero_pidx = (int)t.plain_idx.size();
  dm.T = T.p; dm.T_gstride = 2 * qp; dm.T_pstride = qp; dm.mods = s.d_mods.p;
  dm.N = N; dm.l = l; dm.L = s.L; dm.K = K; dm.nqp = nqp; dm.lt_level = t.level; dm.ng = ng; dm.nbaby = nb;
  dm.g0 = 0; dm.g1 = ng;
  check_mac_tables(t);
  REQUIRE(t.diags.p && t.diags.n >= (t.plain_idx.size() + 1) * dm.diag_stride, "linear transform: diagonal storage missing");
  REQUIRE(t.packed == (t.dense && nb == 16), "linear transform: packed diagonals go with the dense 16-baby kernel");
  for (int b0 = 0; b0 < nb; b0 += 32) {
    dm.b0 = b0; dm.nb_chunk = std::min(32, nb - b0);
    timed("diag_mac", [&] { launch_diag_mac(dm, s.st); });
  }
  // 4. giant groups with a nonzero rotation: ModDown of part 1, decomposition, key product + automorphism + accumulate
  DU64 acc((size_t)2 * qp);
  if (ngk > 0) {
    DU64 t1q((size_t)ngk * (l + 1) * N);
    mod_down(l, T.p + (size_t)gs * 2 * qp + qp, 2 * qp, ngk, t1q.p, (size_t)(l + 1) * N);
    DU64 dg2((size_t)ngk * dn * qp);
    decompose_modup(l, t1q.p, (size_t)(l + 1) * N, ngk, dg2.p, false);
    GiantAccArgs a{};
    a.digits = dg2.p; a.dig_bstride = (size_t)dn * qp; a.key = t.d_gkey.p; a.perm = t.d_gperm.p; a.tg = t.d_tg.p; a.ng = ngk;
    a.own = t1q.p; a.own_bstride = (size_t)(l + 1) * N;
    a.T = T.p; a.T_gstride = 2 * qp; a.T_pstride = qp; a.t_zero = gs ? 0 : -1;
    a.out0 = acc.p; a.out1 = acc.p + qp; a.mods = s.d_mods.p;
    a.N = N; a.l = l; a.L = s.L; a.K = K; a.nqp = nqp; a.dn = dn;
    a.ka = giants_seeded ? t.d_gka.p : nullptr;
    timed("giant_acc", [&] { launch_giant_acc(a, s.st); });
  } else {
    d2d(acc.p, T.p, 2 * qp * 8);
  }
  // 5. final ModDown of both parts (with the first rescale when the result is
  // to be returned rescaled)
  const double sc = ct.scale * t.scale;
  REQUIRE(!rescale || l >= 1, "cannot rescale: ciphertext already at level 0");
  const int nres = rescale ? lattigo_rescale_count(sc, l) : 0;
  if (nres == 0) {
    auto out = new_ct(l, sc); out->logslots = ct.logslots;
    mod_down(l, acc.p, qp, 2, out->d.p, (size_t)(l + 1) * N);
    return out;
  }
  auto out = new_ct(l - 1, sc / (double)s.mod[l]); out->logslots = ct.logslots;
  mod_down_rescale(l, acc.p, qp, 2, out->d.p, (size_t)l * N);
  for (int i = 1; i < nres; i++) out = rescale_ct(*out);
  return out;
}
// MultiplyByDiagMatrix (naive, N1 = 0)
std::unique_ptr<Cipher> eval_lt_naive(const LinTrans& t, const Cipher& ct) {
  Scheme& s = sch();
  const int N = s.N, K = s.K;
  const int l = std::min(ct.level, t.level), nqp = l + 1 + K, dn = (l + 1 + K - 1) / K;
  const size_t qp = (size_t)nqp * N;
  const u64* c0 = ct.d.p;
  const u64* c1 = ct.d.p + (size_t)(ct.level + 1) * N;
  DU64 digits((size_t)dn * qp);
  decompose_modup(l, c1, 0, 1, digits.p, false);
  DU64 pc((size_t)(l + 1) * N);
  launch_mul_const(pc.p, c0, 0, 1, rows_q(l), s.pmod_w.p, s.pmod_wp.p, s.d_mods.p, N, s.st);
  std::vector<int> nz; int zero_p = -1;
  for (size_t i = 0; i < t.plain_idx.size(); i++) { if ((t.plain_idx[i] & (t.slots - 1)) == 0) zero_p = (int)i; else nz.push_back((int)i); }
  DU64 acc((size_t)2 * qp);
  HCHECK(hipMemsetAsync(acc.p, 0, acc.bytes(), s.st));
  const size_t dstride = (size_t)(t.level + 1 + K) * N;
  if (!nz.empty()) {
    const int n = (int)nz.size();
    std::vector<const u64*> kh(n); std::vector<const uint32_t*> ph(n);
    for (int i = 0; i < n; i++) { u64 ge = galois_element(t.plain_idx[nz[i]] & (t.slots - 1)); kh[i] = key_ptr(ge, true); ph[i] = perm_for(ge); }
    DevArray<const u64*> kp(n); DevArray<const uint32_t*> pp(n);
    upload(kp.p, kh.data(), n); upload(pp.p, ph.data(), n);
    DU64 R((size_t)n * 2 * qp);
    KeyMacArgs a{};
    a.digits = digits.p; a.key = kp.p; a.perm = pp.p; a.add0 = pc.p;
    a.own = c1; a.own_bstride = 0;
    a.out0 = R.p; a.out1 = R.p + qp; a.out_bstride = 2 * qp; a.mods = s.d_mods.p;
    a.N = N; a.l = l; a.L = s.L; a.K = K; a.nqp = nqp; a.dn = dn;
    launch_keymac(a, n, s.st);
    for (int i = 0; i < n; i++) {
      const u64* dp = t.diags.p + (size_t)nz[i] * dstride;
      // the diagonal's P rows sit after its own Q rows (level t.level); multiply Q and P parts separately
      launch_mont_mul(acc.p, qp, R.p + (size_t)i * 2 * qp, qp, dp, 0, 2, rows_q(l), s.d_mods.p, N, true, s.st);
      launch_mont_mul(acc.p + (size_t)(l + 1) * N, qp, R.p + (size_t)i * 2 * qp + (size_t)(l + 1) * N, qp, dp + (size_t)(t.level + 1) * N, 0, 2,
                      RowMap{K, 0, 0, s.L, 0, 0}, s.d_mods.p, N, true, s.st);
    }
  }
  auto out = new_ct(l, ct.scale * t.scale); out->logslots = ct.logslots;
  mod_down(l, acc.p, qp, 2, out->d.p, (size_t)(l + 1) * N);
  if (zero_p >= 0) {
    const u64* dp = t.diags.p + (size_t)zero_p * dstride;
    launch_mont_mul(out->d.p, (size_t)(l + 1) * N, c0, 0, dp, 0, 1, rows_q(l), s.d_mods.p, N, true, s.st);
    launch_mont_mul(out->d.p + (size_t)(l + 1) * N, 0, c1, 0, dp, 0, 1, rows_q(l), s.d_mods.p, N, true, s.st);
  }
  return out;
}

// ============================================================================
// encrypt / decrypt
// ============================================================================
std::unique_ptr<Cipher> encrypt_pt(const Plain& pt) {
  Scheme& s = sch();
  REQUIRE(s.has_pk, "public key not generated");
  const int l = pt.level, N = s.N, nm = s.L + s.K, nr = l + 2;
  const u64 enc = s.enc_counter++;
  std::vector<int8_t> u = ternary_hw(s.seed, ST_ENC_U(enc), N, s.h);
  DevArray<int8_t> du(N); upload(du.p, u.data(), N);
  RowMap rm{nr, l + 1, 0, s.L, 0, 0};
  DU64 uq((size_t)nr * N), pk((size_t)2 * nr * N), tt((size_t)2 * nr * N);
  launch_signed_rows(uq.p, rm, du.p, s.d_mods.p, N, s.st);
  ntt(uq.p, 0, 1, rm, true);
  for (int p = 0; p < 2; p++) {
    d2d(pk.p + (size_t)p * nr * N, s.pkR.p + (size_t)p * nm * N, (size_t)(l + 1) * N * 8);
    d2d(pk.p + (size_t)p * nr * N + (size_t)(l + 1) * N, s.pkR.p + (size_t)p * nm * N + (size_t)s.L * N, (size_t)N * 8);
  }
  launch_mont_mul(tt.p, (size_t)nr * N, uq.p, 0, pk.p, (size_t)nr * N, 2, rm, s.d_mods.p, N, false, s.st);
  ntt(tt.p, (size_t)nr * N, 2, rm, false);
  launch_sample_cbd(tt.p, rm, s.seed, ST_ENC_E0(enc), s.d_mods.p, N, true, s.st);
  launch_sample_cbd(tt.p + (size_t)nr * N, rm, s.seed, ST_ENC_E1(enc), s.d_mods.p, N, true, s.st);
  // ModDown from Q + {p_0} in the coefficient domain
  DU64 ext((size_t)2 * (l + 1) * N);
  BConvHost& bt = bconv_table(s.L, s.L + 1);
  launch_bconv(tt.p + (size_t)(l + 1) * N, (size_t)nr * N, 1, bt.dtab.p, ext.p, (size_t)(l + 1) * N, 2, rows_q(l), s.d_mods.p, N, false, s.st);
  auto out = new_ct(l, pt.scale); out->logslots = pt.logslots;
  launch_moddown_combine(out->d.p, (size_t)(l + 1) * N, tt.p, (size_t)nr * N, ext.p, (size_t)(l + 1) * N, nullptr, 0, 0, nullptr,
                         s.p0inv_w.p, s.p0inv_wp.p, l + 1, 2, s.d_mods.p, N, s.st);
  ntt(out->d.p, (size_t)(l + 1) * N, 2, rows_q(l), true);
  launch_add(out->d.p, out->d.p, pt.d.p, 0, 1, rows_q(l), s.d_mods.p, N, false, s.st);
  sync();
  return out;
}
// Seeded secret-key encryption (the compressed upload of
// orion/backend/cheddar/ext/cheddar_pybind.cu:627-660): a is expanded from the
// client's seed directly in the NTT domain, a[i][x] = uniform(rand64(seed,
// ST_SEED_A, i*N + x)) mod q_i, so a server that received only (b, seed)
// rebuilds it with expand_seeded_a; b = -a*s + e + m.
void expand_seeded_a(Cipher& c, u64 seed) {
  Scheme& s = sch();
  launch_sample_uniform(c.d.p + (size_t)(c.level + 1) * s.N, rows_q(c.level), seed, ST_SEED_A, s.d_mods.p, s.N, s.st);
}
std::unique_ptr<Cipher> encrypt_seeded(const Plain& pt, u64 seed) {
  Scheme& s = sch();
  REQUIRE(s.has_sk, "secret key not generated");
  const int l = pt.level, N = s.N;
  const u64 enc = s.enc_counter++;
  auto out = new_ct(l, pt.scale); out->logslots = pt.logslots;
  u64* b = out->d.p;
  expand_seeded_a(*out, seed);
  launch_sample_cbd(b, rows_q(l), s.seed, ST_SEED_E(enc), s.d_mods.p, N, false, s.st);
  ntt(b, 0, 1, rows_q(l), true);
  DU64 as((size_t)(l + 1) * N);
  launch_mont_mul(as.p, 0, b + (size_t)(l + 1) * N, 0, s.sR.p, 0, 1, rows_q(l), s.d_mods.p, N, false, s.st);
  launch_add(b, b, as.p, 0, 1, rows_q(l), s.d_mods.p, N, true, s.st);
  launch_add(b, b, pt.d.p, 0, 1, rows_q(l), s.d_mods.p, N, false, s.st);
  sync();
  return out;
}
std::unique_ptr<Plain> decrypt_ct(const Cipher& ct) {
  Scheme& s = sch();
  REQUIRE(s.has_sk, "secret key not generated");
  const int l = ct.level, N = s.N;
  auto p = std::make_unique<Plain>();
  p->level = l; p->scale = ct.scale; p->logslots = ct.logslots;
  p->d = DU64((size_t)(l + 1) * N);
  d2d(p->d.p, ct.d.p, (size_t)(l + 1) * N * 8);
  launch_mont_mul(p->d.p, 0, ct.d.p + (size_t)(l + 1) * N, 0, s.sR.p, 0, 1, rows_q(l), s.d_mods.p, N, true, s.st);
  sync();
  return p;
}

std::unique_ptr<Plain> encode_values(const float* v, int n, int level, double scale) {
  Scheme& s = sch();
  REQUIRE(level >= 0 && level < s.L, "invalid level");
  REQUIRE(n >= 0 && n <= s.N / 2, "too many values for the slot count");
  auto p = std::make_unique<Plain>();
  p->level = level; p->scale = scale; p->logslots = s.logN - 1;
  p->d = DU64((size_t)(level + 1) * s.N);
  // the load kernel reads a full slots-wide row: pad the values with zeros
  std::vector<float> buf((size_t)s.N / 2, 0.0f);
  std::copy(v, v + n, buf.begin());
  encode_device(buf.data(), buf.size(), {EncodeSrc{0, 0}}, n, scale, rows_q(level), p->d.p, 0);
  return p;
}
// complex slot values, interleaved (re, im) pairs as EncodeComplex passes them
std::unique_ptr<Plain> encode_complex_values(const float* v, int n, int level, double scale) {
  Scheme& s = sch();
  REQUIRE(level >= 0 && level < s.L, "invalid level");
  REQUIRE(n >= 0 && n <= s.N / 2, "too many values for the slot count");
  auto p = std::make_unique<Plain>();
  p->level = level; p->scale = scale; p->logslots = s.logN - 1;
  p->d = DU64((size_t)(level + 1) * s.N);
  std::vector<float> buf((size_t)s.N, 0.0f);
  std::copy(v, v + 2 * (size_t)n, buf.begin());
  encode_device(buf.data(), buf.size(), {EncodeSrc{0, 0}}, n, scale, rows_q(level), p->d.p, 0, true);
  return p;
}
std::vector<double> decode_pt(const Plain& p, std::vector<double>* imag = nullptr) {
  Scheme& s = sch();
  const int N = s.N, l = p.level;
  DU64 tmp((size_t)(l + 1) * N);
  d2d(tmp.p, p.d.p, tmp.bytes());
  ntt(tmp.p, 0, 1, rows_q(l), false);
  std::vector<u64> coef((size_t)(l + 1) * N);
  download(coef.data(), tmp.p, coef.size());
  return decode_host(coef, l, p.scale, imag);
}

template <class T> T* c_array(const std::vector<T>& v) {
  T* p = (T*)std::malloc(std::max<size_t>(1, v.size()) * sizeof(T));
  if (!p) throw Error("out of host memory");
  if (!v.empty()) std::memcpy(p, v.data(), v.size() * sizeof(T));
  return p;
}
unsigned long scale_to_ulong(double sc) { if (!(sc < 18446744073709551616.0)) return ~0UL; return sc < 0 ? 0UL : (unsigned long)sc; }

// ---- binary wire format --------------------------------------------------------
// The layout of Lattigo v6's WriteTo for the objects Orion serializes
// (keygenerator.go:38-58, lineartransform.go:130-193), little-endian u64 words:
//   ring.Poly    rows, then per row: N, N coefficients
//   ringqp.Poly  ring.Poly over Q, then ring.Poly over P
//   SecretKey    ringqp.Poly over the whole QP basis
//   GaloisKey    galois element, NthRoot (2N), base-two decomposition (0),
//                dnum, then per digit: 1, 2, (b, a) as ringqp.Poly
//   diagonal     ringqp.Poly at the transform's level
// Everything stays in the NTT domain and in Montgomery form (x * 2^64 mod q).
// Ciphertexts and plaintexts (no counterpart in the reference, which never
// serializes them) follow the field order of Lattigo v6's rlwe.Element:
// metadata, then the vector of polynomials:
//   metadata     scale (IEEE-754 binary64 bits), log2 slots, flags
//                (bit 0 batched, bit 1 NTT domain, bit 2 Montgomery form)
//   vector       count (2 ciphertext, 1 plaintext), then count ring.Poly
// with standard representatives in the NTT domain (flags 0b011).
constexpr u64 WIRE_ELEM_FLAGS = 0x3;
struct Wire {
  std::vector<uint8_t> b;
  void u64v(u64 x) { for (int i = 0; i < 8; i++) b.push_back((uint8_t)(x >> (8 * i))); }
  void words(const u64* p, size_t n) {
    size_t o = b.size(); b.resize(o + 8 * n);
    for (size_t i = 0; i < n; i++) for (int k = 0; k < 8; k++) b[o + 8 * i + k] = (uint8_t)(p[i] >> (8 * k));
  }
  void poly(const u64* rows, int nrows, int N) { u64v((u64)nrows); for (int r = 0; r < nrows; r++) { u64v((u64)N); words(rows + (size_t)r * N, N); } }
  void qp(const u64* rows, int nq, int K, int N) { poly(rows, nq, N); poly(rows + (size_t)nq * N, K, N); }
};
struct WireIn {
  const uint8_t* p; size_t n, off = 0;
  u64 u64v() {
    REQUIRE(off + 8 <= n, "serialized data truncated");
    u64 x = 0; for (int i = 0; i < 8; i++) x |= (u64)p[off + i] << (8 * i);
    off += 8; return x;
  }
  void words(u64* out, size_t cnt) {
    REQUIRE(off + 8 * cnt <= n, "serialized data truncated");
    for (size_t i = 0; i < cnt; i++) { u64 x = 0; for (int k = 0; k < 8; k++) x |= (u64)p[off + 8 * i + k] << (8 * k); out[i] = x; }
    off += 8 * cnt;
  }
  void poly(u64* rows, int nrows, int N, const std::vector<u64>& mods, int m0) {
    REQUIRE(u64v() == (u64)nrows, "serialized polynomial has the wrong number of limbs");
    for (int r = 0; r < nrows; r++) {
      REQUIRE(u64v() == (u64)N, "serialized polynomial has the wrong ring degree");
      u64* row = rows + (size_t)r * N; words(row, N);
      for (int x = 0; x < N; x++) REQUIRE(row[x] < mods[m0 + r], "serialized coefficient not reduced");
    }
  }
  void qp(u64* rows, int nq, int K, int N, const std::vector<u64>& mods, int Lfull) {
    poly(rows, nq, N, mods, 0);
    poly(rows + (size_t)nq * N, K, N, mods, Lfull);
  }
  void end() { REQUIRE(off == n, "trailing bytes after the serialized object"); }
};
// the moduli of a QP polynomial at level l are q_0..q_l then p_0..p_{K-1}
std::vector<u64> qp_mods(int l) {
  Scheme& s = sch();
  std::vector<u64> m(s.mod.begin(), s.mod.begin() + l + 1);
  m.insert(m.end(), s.mod.begin() + s.L, s.mod.end());
  return m;
}
ArrayResultByte bytes_result(const std::vector<uint8_t>& v) {
  ArrayResultByte r;
  r.Data = (char*)c_array(v); r.Length = v.size();
  return r;
}
std::vector<uint8_t> serialize_element(const u64* d, int npoly, int level, double scale, int logslots) {
  Scheme& s = sch();
  const int N = s.N;
  std::vector<u64> h((size_t)npoly * (level + 1) * N);
  download(h.data(), d, h.size());
  Wire w;
  u64 bits;
  std::memcpy(&bits, &scale, 8);
  w.u64v(bits); w.u64v((u64)logslots); w.u64v(WIRE_ELEM_FLAGS);
  w.u64v((u64)npoly);
  for (int p = 0; p < npoly; p++) w.poly(h.data() + (size_t)p * (level + 1) * N, level + 1, N);
  return w.b;
}
// parses an element written by serialize_element; returns its words
// (npoly x rows x N), level, scale and log2 slots
std::vector<u64> parse_element(const unsigned char* data, size_t len, int npoly, int& level, double& scale, int& logslots) {
  Scheme& s = sch();
  const int N = s.N;
  REQUIRE(data, "no data");
  WireIn in{data, len};
  const u64 bits = in.u64v();
  std::memcpy(&scale, &bits, 8);
  REQUIRE(std::isfinite(scale) && scale > 0, "serialized scale is not a positive number");
  const u64 ls = in.u64v();
  REQUIRE(ls >= 1 && ls <= (u64)(s.logN - 1), "serialized slot count does not fit the ring");
  logslots = (int)ls;
  REQUIRE(in.u64v() == WIRE_ELEM_FLAGS, "serialized element is not in the NTT domain with standard representatives");
  REQUIRE(in.u64v() == (u64)npoly, npoly == 2 ? "serialized element is not a degree-1 ciphertext" : "serialized element is not a plaintext");
  // the row count of the first polynomial fixes the level
  REQUIRE(in.off + 8 <= in.n, "serialized data truncated");
  u64 rows = 0;
  for (int i = 0; i < 8; i++) rows |= (u64)in.p[in.off + i] << (8 * i);
  REQUIRE(rows >= 1 && rows <= (u64)s.L, "serialized element has more limbs than the Q chain");
  level = (int)rows - 1;
  std::vector<u64> h((size_t)npoly * rows * N);
  for (int p = 0; p < npoly; p++) in.poly(h.data() + (size_t)p * rows * N, (int)rows, N, s.mod, 0);
  in.end();
  return h;
}
std::vector<uint8_t> serialize_galois_key(u64 galel, const DU64& key) {
  Scheme& s = sch();
  const int N = s.N, nm = s.L + s.K;
  std::vector<u64> h((size_t)s.dnum * 2 * nm * N);
  download(h.data(), key.p, h.size());
  Wire w;
  w.u64v(galel); w.u64v(2 * (u64)N); w.u64v(0); w.u64v((u64)s.dnum);
  for (int d = 0; d < s.dnum; d++) {
    w.u64v(1); w.u64v(2);
    for (int p = 0; p < 2; p++) w.qp(h.data() + ((size_t)d * 2 + p) * nm * N, s.L, s.K, N);
  }
  return w.b;
}

}  // namespace

// ============================================================================
// C ABI
// ============================================================================
extern "C" {

const char* GetLastError(void) { return g_err.c_str(); }
void SetSchemeSeed(uint64_t seed) { g_seed_override = seed; g_seed_set = true; }

int NewScheme(int logN, int* logQ, int lenQ, int* logP, int lenP, int logScale, int h, const char* ringType,
              const char* keysPath, const char* ioMode) {
  return guard([&] {
    (void)keysPath; (void)ioMode;
    REQUIRE(ringType && std::string(ringType) == "standard", "only the standard ring is supported by the hip backend");
    std::vector<int> lq(logQ, logQ + lenQ), lp(logP, logP + lenP);
    std::vector<u64> q, p;
    gen_primes(logN, lq, lp, q, p);
    u64 seed = g_seed_override;
    if (!g_seed_set) { FILE* f = std::fopen("/dev/urandom", "rb"); if (f) { if (std::fread(&seed, 8, 1, f) != 1) seed = 0; std::fclose(f); } }
    build_scheme(logN, q, p, logScale, h, seed);
    return 0;
  });
}
int NewSchemeWithModuli(int logN, const uint64_t* q, int lenQ, const uint64_t* p, int lenP, int logScale, int h, uint64_t seed) {
  return guard([&] {
    build_scheme(logN, std::vector<u64>(q, q + lenQ), std::vector<u64>(p, p + lenP), logScale, h, seed);
    return 0;
  });
}
int DeleteScheme(void) {
  return guard([&] {
    if (S) { delete S; S = nullptr; }
    for (auto& kv : g_scratch_use) kv.second.last = nullptr;  // its streams are gone
    if (g_pool) g_pool->release_all();
    return 0;
  });
}
int GeneratePrimes(int logN, const int* logQ, int lenQ, const int* logP, int lenP, uint64_t* q, uint64_t* p) {
  return guard([&] {
    std::vector<u64> qq, pp;
    gen_primes(logN, std::vector<int>(logQ, logQ + lenQ), std::vector<int>(logP, logP + lenP), qq, pp);
    std::copy(qq.begin(), qq.end(), q); std::copy(pp.begin(), pp.end(), p);
    return 0;
  });
}

// ---- keys ----
int NewKeyGenerator(void) { return guard([&] { sch(); return 0; }); }
int GenerateSecretKey(void) { return guard([&] { gen_secret(); return 0; }); }
int GeneratePublicKey(void) { return guard([&] { gen_public(); return 0; }); }
int GenerateRelinearizationKey(void) { return guard([&] { ensure_relin_key(); return 0; }); }
int GenerateEvaluationKeys(void) { return guard([&] { sch(); return 0; }); }

// ---- encoder ----
int NewEncoder(void) { return guard([&] { sch().encoder = true; return 0; }); }
int Encode(const float* values, int lenValues, int level, unsigned long scale) {
  return guard([&] {
    return push_pt(encode_values(values, lenValues, level, (double)scale));
  });
}
ArrayResultFloat Decode(int plaintextID) {
  ArrayResultFloat r{nullptr, 0};
  guard([&] {
    std::vector<double> v = decode_pt(get_pt(plaintextID));
    std::vector<float> f(v.begin(), v.end());
    r.Data = c_array(f); r.Length = f.size();
    return 0;
  });
  return r;
}
int DecodeDouble(int plaintextID, double* out, int len) {
  return guard([&] {
    std::vector<double> v = decode_pt(get_pt(plaintextID));
    REQUIRE(len >= (int)v.size(), "output buffer too small");
    std::copy(v.begin(), v.end(), out);
    return (int)v.size();
  });
}

int EncodeComplex(const float* values, int lenValues, int level, unsigned long scale) {
  return guard([&] {
    REQUIRE(lenValues % 2 == 0, "complex values come as (re, im) pairs");
    return push_pt(encode_complex_values(values, lenValues / 2, level, (double)scale));
  });
}
ArrayResultFloat DecodeComplex(int plaintextID) {
  ArrayResultFloat r{nullptr, 0};
  guard([&] {
    std::vector<double> im;
    std::vector<double> re = decode_pt(get_pt(plaintextID), &im);
    std::vector<float> f(2 * re.size());
    for (size_t i = 0; i < re.size(); i++) { f[2 * i] = (float)re[i]; f[2 * i + 1] = (float)im[i]; }
    r.Data = c_array(f); r.Length = f.size();
    return 0;
  });
  return r;
}

// ---- encryptor ----
int NewEncryptor(void) { return guard([&] { sch().encryptor = true; return 0; }); }
int NewDecryptor(void) { return guard([&] { sch().decryptor = true; return 0; }); }
int Encrypt(int plaintextID) { return guard([&] { return push_ct(encrypt_pt(get_pt(plaintextID))); }); }
int Decrypt(int ciphertextID) { return guard([&] { return push_pt(decrypt_ct(get_ct(ciphertextID))); }); }
int EncryptSeeded(int plaintextID, unsigned long long seed) {
  return guard([&] { return push_ct(encrypt_seeded(get_pt(plaintextID), (u64)seed)); });
}
int DropAx(int ciphertextID) {
  return guard([&] {
    Scheme& s = sch(); Cipher& c = get_ct(ciphertextID);
    HCHECK(hipMemsetAsync(c.d.p + (size_t)(c.level + 1) * s.N, 0, (size_t)(c.level + 1) * s.N * 8, s.st));
    sync();
    return 0;
  });
}
int ExpandSeededAx(int ciphertextID, unsigned long long seed) {
  return guard([&] { expand_seeded_a(get_ct(ciphertextID), (u64)seed); sync(); return 0; });
}
double GetCiphertextBytes(int ciphertextID) {
  double v = -1; guard([&] { const Cipher& c = get_ct(ciphertextID); v = 2.0 * (c.level + 1) * sch().N * 8; return 0; }); return v;
}
double GetCiphertextBxBytes(int ciphertextID) {
  double v = -1; guard([&] { const Cipher& c = get_ct(ciphertextID); v = 1.0 * (c.level + 1) * sch().N * 8; return 0; }); return v;
}
int SetEncryptionCounter(uint64_t v) { return guard([&] { sch().enc_counter = v; return 0; }); }

// ---- evaluator ----
int AddRotationKey(int rotation) {
  return guard([&] { u64 ge = galois_element(rotation); ensure_galois_key(ge); sch().rot_keys.insert(ge); return 0; });
}
int NewEvaluator(void) {
  return guard([&] {
    Scheme& s = sch();
    s.evaluator = true;
    for (int i = 1; i < s.N / 2; i *= 2) { u64 ge = galois_element(i); ensure_galois_key(ge); s.rot_keys.insert(ge); }
    u64 conj = 2 * (u64)s.N - 1;
    ensure_galois_key(conj); s.rot_keys.insert(conj);
    return 0;
  });
}
int Rotate(int ctID, int amount) {
  return guard([&] {
    AddRotationKey(amount);
    Cipher& c = get_ct(ctID);
    auto r = automorphism(c, galois_element(amount), false);
    c.d = std::move(r->d);
    return ctID;
  });
}
int RotateNew(int ctID, int amount) {
  return guard([&] {
    u64 ge = galois_element(amount); ensure_galois_key(ge); sch().rot_keys.insert(ge);
    return push_ct(automorphism(get_ct(ctID), ge, false));
  });
}
// [ext] ct <- ct + Rotate(ct, amount): one step of a Linear's output fold
// (linear.py:115-117, `out += out.roll(k)`), the add done in the key
// switch's ModDown epilogue instead of a separate pass.  The sum is formed in
// a new buffer (the epilogue's scattered stores cannot overwrite the words
// they read) that then replaces the ciphertext's own.  Same words as
// RotateNew + AddCiphertext.
int RotateAdd(int ctID, int amount) {
  return guard([&] {
    u64 ge = galois_element(amount); ensure_galois_key(ge); sch().rot_keys.insert(ge);
    Cipher& ct = get_ct(ctID);
    const u64* key = key_ptr(ge, false);
    auto out = new_ct(ct.level, ct.scale);
    timed("rotate", [&] { automorphism_core(ct, ge, key, perm_inv_for(ge), out->d.p, nullptr, ct.d.p); });
    std::swap(ct.d, out->d);
    return ctID;
  });
}
// RotateNew into an existing ciphertext with no allocation: the key switch's
// temporaries live in the device scratch array, the automorphism tables and
// basis-conversion tables were built with the key and the scheme.  The
// rotation key must exist already.  A call on the other stream of the
// scheme waits for the previous call's key switch; calls from several host
// threads or processes sharing the GPU race on the array.
int RotateInto(int ctID, int amount, int outID) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(ctID != outID, "RotateInto: the output must be another ciphertext than the input");
    const Cipher& c = get_ct(ctID);
    Cipher& o = get_ct(outID);
    const u64 ge = galois_element(amount);
    REQUIRE(s.rot_keys.count(ge) && s.gkeys.count(ge),
            "RotateInto: no rotation key for this amount (AddRotationKey or RotateNew generates it)");
    const size_t need = automorphism_ws_words(c.level);
    REQUIRE(need <= SCRATCH_WORDS, "RotateInto: the key switch needs " + std::to_string(need * 8) +
                                       " bytes of scratch at this level, more than the " +
                                       std::to_string(SCRATCH_WORDS * 8) + " bytes available");
    REQUIRE(o.d.n >= (size_t)2 * (c.level + 1) * s.N, "RotateInto: the output ciphertext is too small for the input's level");
    u64* ws = scratch_ptr();
    ScratchUse& use = scratch_use();
    // the previous call's key switch, if queued on another stream, is done
    // with the array before this one starts
    if (use.last && use.last != s.st) HCHECK(hipStreamWaitEvent(s.st, use.ev, 0));
    {
      // the buffer cache refuses to hand out memory until the key switch is queued
      struct NoAlloc { NoAlloc() { g_pool->forbid++; } ~NoAlloc() { g_pool->forbid--; } } guard_alloc;
      automorphism_core(c, ge, s.gkeys.at(ge)->p, perm_inv_cached(ge), o.d.p, ws);
    }
    HCHECK(hipEventRecord(use.ev, s.st));
    use.last = s.st;
    o.level = c.level; o.scale = c.scale; o.logslots = c.logslots;
    return outID;
  });
}
int Conjugate(int ctID) {
  return guard([&] { Scheme& s = sch(); u64 ge = 2 * (u64)s.N - 1; ensure_galois_key(ge); s.rot_keys.insert(ge);
    Cipher& c = get_ct(ctID); auto r = automorphism(c, ge, false); c.d = std::move(r->d); return ctID; });
}
int ConjugateNew(int ctID) {
  return guard([&] { Scheme& s = sch(); u64 ge = 2 * (u64)s.N - 1; ensure_galois_key(ge); s.rot_keys.insert(ge);
    return push_ct(automorphism(get_ct(ctID), ge, false)); });
}
int Rescale(int ctID) {
  return guard([&] { Cipher& c = get_ct(ctID); auto r = rescale_lattigo(c); c = std::move(*r); return ctID; });
}
// As the reference wrapper (evaluator.go RescaleNew): rescales the input in place, returns a copy.
int RescaleNew(int ctID) {
  return guard([&] { Cipher& c = get_ct(ctID); auto r = rescale_lattigo(c); c = std::move(*r); return push_ct(copy_ct(c)); });
}
int AddCiphertext(int a, int b) { return guard([&] { add_inplace(get_ct(a), get_ct(b), false); return a; }); }
int AddCiphertextNew(int a, int b) { return guard([&] { auto c = copy_ct(get_ct(a)); add_inplace(*c, get_ct(b), false); return push_ct(std::move(c)); }); }
int SubCiphertext(int a, int b) { return guard([&] { add_inplace(get_ct(a), get_ct(b), true); return a; }); }
int SubCiphertextNew(int a, int b) { return guard([&] { auto c = copy_ct(get_ct(a)); add_inplace(*c, get_ct(b), true); return push_ct(std::move(c)); }); }
int AddPlaintext(int ct, int pt) { return guard([&] { add_plain_inplace(get_ct(ct), get_pt(pt), false); return ct; }); }
int AddPlaintextNew(int ct, int pt) { return guard([&] { auto c = copy_ct(get_ct(ct)); add_plain_inplace(*c, get_pt(pt), false); return push_ct(std::move(c)); }); }
int MulPlaintext(int ct, int pt) {
  return guard([&] { Cipher& c = get_ct(ct); auto r = mul_plain_ct(c, get_pt(pt)); c = std::move(*r); return ct; });
}
int MulPlaintextNew(int ct, int pt) { return guard([&] { return push_ct(mul_plain_ct(get_ct(ct), get_pt(pt))); }); }
int MulScalarInt(int ct, int k) { return guard([&] { mul_int_inplace(get_ct(ct), k); return ct; }); }
int MulScalarIntNew(int ct, int k) { return guard([&] { auto c = copy_ct(get_ct(ct)); mul_int_inplace(*c, k); return push_ct(std::move(c)); }); }
int MulScalarFloat(int ct, float v) { return guard([&] { mul_float_inplace(get_ct(ct), (double)v); return ct; }); }
int MulScalarFloatNew(int ct, float v) {
  return guard([&] { auto c = copy_ct(get_ct(ct)); mul_float_inplace(*c, (double)v); return push_ct(std::move(c)); });
}
int AddScalar(int ct, float v) { return guard([&] { add_const_inplace(get_ct(ct), (double)v, false); return ct; }); }
int AddScalarNew(int ct, float v) {
  return guard([&] { auto c = copy_ct(get_ct(ct)); add_const_inplace(*c, (double)v, false); return push_ct(std::move(c)); });
}
int SubScalar(int ct, float v) { return guard([&] { add_const_inplace(get_ct(ct), (double)v, true); return ct; }); }
int SubScalarNew(int ct, float v) {
  return guard([&] { auto c = copy_ct(get_ct(ct)); add_const_inplace(*c, (double)v, true); return push_ct(std::move(c)); });
}
// multiplication by i = by the monomial X^(N/2), key-free, in the NTT domain
void mul_i_inplace(Cipher& c) {
  Scheme& s = sch();
  const size_t ps = (size_t)(c.level + 1) * s.N;
  launch_mul_i(c.d.p, c.d.p, ps, 2, rows_q(c.level), s.iu.p, s.iup.p, s.niu.p, s.niup.p, s.d_mods.p, s.N, s.st);
}
int MulImaginaryUnit(int ct) { return guard([&] { mul_i_inplace(get_ct(ct)); return ct; }); }
int MulImaginaryUnitNew(int ct) { return guard([&] { auto c = copy_ct(get_ct(ct)); mul_i_inplace(*c); return push_ct(std::move(c)); }); }
int Negate(int ct) { return guard([&] { auto c = copy_ct(get_ct(ct)); mul_float_inplace(*c, -1.0); return push_ct(std::move(c)); }); }
int MulRelinCiphertext(int a, int b) {
  return guard([&] { Cipher& c = get_ct(a); auto r = mul_relin_ct(c, get_ct(b), false); c = std::move(*r); return a; });
}
int MulRelinCiphertextNew(int a, int b) { return guard([&] { return push_ct(mul_relin_ct(get_ct(a), get_ct(b), false)); }); }

// ---- polynomial evaluator ----
int NewPolynomialEvaluator(void) { return guard([&] { sch(); return 0; }); }
int GenerateMonomial(const float* coeffs, int lenCoeffs) {
  return guard([&] {
    REQUIRE(coeffs && lenCoeffs >= 1, "empty polynomial");
    Scheme& s = sch();
    int id = s.poly_ids.take();
    s.polys[id] = std::vector<double>(coeffs, coeffs + lenCoeffs);
    return id;
  });
}
// Chebyshev basis on [-1, 1] (T0 = 1, T1 = x, T2 = 2x^2 - 1, T3 = 4x^3 - 3x),
// kept as its monomial form (degree <= 3)
int GenerateChebyshev(const float* coeffs, int lenCoeffs) {
  return guard([&] {
    REQUIRE(coeffs && lenCoeffs >= 1, "empty polynomial");
    REQUIRE(lenCoeffs <= 4, "the hip backend evaluates polynomials of degree <= 3");
    double c[4] = {0, 0, 0, 0};
    for (int i = 0; i < lenCoeffs; i++) c[i] = coeffs[i];
    std::vector<double> m = {c[0] - c[2], c[1] - 3.0 * c[3], 2.0 * c[2], 4.0 * c[3]};
    m.resize(lenCoeffs);
    Scheme& s = sch();
    int id = s.poly_ids.take();
    s.polys[id] = m;
    return id;
  });
}
int EvaluatePolynomial(int ctInID, int polyID, unsigned long outScale) {
  return guard([&] {
    Scheme& s = sch();
    auto it = s.polys.find(polyID);
    REQUIRE(it != s.polys.end(), "polynomial not found: " + std::to_string(polyID));
    return push_ct(eval_poly_ct(get_ct(ctInID), it->second, (double)outScale));
  });
}
int SubPlaintext(int ct, int pt) { return guard([&] { add_plain_inplace(get_ct(ct), get_pt(pt), true); return ct; }); }
int SubPlaintextNew(int ct, int pt) { return guard([&] { auto c = copy_ct(get_ct(ct)); add_plain_inplace(*c, get_pt(pt), true); return push_ct(std::move(c)); }); }

// ---- linear transforms ----
int NewLinearTransformEvaluator(void) { return guard([&] { sch().lteval = true; return 0; }); }
int GenerateLinearTransform(const int* diagIdxs, int diagIdxsLen, const float* diagData, int diagDataLen, int level,
                            float bsgsRatio, const char* ioMode) {
  return guard([&] {
    const std::string mode = ioMode ? ioMode : "none";
    REQUIRE(mode == "none" || mode == "save" || mode == "load", "io_mode must be 'none', 'save' or 'load'");
    return generate_lt(diagIdxs, diagIdxsLen, diagData, diagDataLen, level, bsgsRatio, mode == "load");
  });
}
int EvaluateLinearTransform(int transformID, int ctxtID) {
  return guard([&] {
    LinTrans& t = get_lt(transformID);
    Cipher& c = get_ct(ctxtID);
    REQUIRE(std::all_of(t.resident.begin(), t.resident.end(), [](char r) { return r != 0; }),
            "plaintext diagonals not loaded (LoadPlaintextDiagonal)");
    const bool rescale = sch().lt_prerescale;
    auto out = t.naive ? eval_lt_naive(t, c) : eval_lt_bsgs(t, c, rescale);
    if (rescale && t.naive) out = rescale_lattigo(*out);
    return push_ct(std::move(out));
  });
}
int SetLinearTransformPrerescale(int on) {
  return guard([&] { sch().lt_prerescale = on != 0; return 0; });
}
int GetLinearTransformPrerescale() { return S && S->lt_prerescale ? 1 : 0; }
ArrayResultInt GetLinearTransformRotationKeys(int transformID) {
  ArrayResultInt r{nullptr, 0};
  guard([&] {
    std::vector<int> ge;
    for (int k : lt_rotations(get_lt(transformID))) ge.push_back((int)galois_element(k));
    r.Data = c_array(ge); r.Length = ge.size();
    return 0;
  });
  return r;
}
int GenerateLinearTransformRotationKey(int galEl) {
  return guard([&] { ensure_galois_key((u64)(unsigned)galEl); sch().lt_keys.insert((u64)(unsigned)galEl); return 0; });
}
int DeleteLinearTransform(int id) {
  return guard([&] { Scheme& s = sch(); sync(); if (s.lts.erase(id)) s.lt_ids.give(id); return 0; });
}
int RemoveRotationKeys(void) {
  return guard([&] {
    // the transforms lose their keys; keys that Rotate also uses stay (lineartransform.go:203-211)
    Scheme& s = sch();
    sync();
    for (u64 g : s.lt_keys) if (!s.rot_keys.count(g)) s.gkeys.erase(g);
    s.lt_keys.clear();
    for (auto& kv : s.lts) kv.second->ptrs_ready = false;
    return 0;
  });
}

// ---- serialization (io_mode save / load) ----
ArrayResultByte SerializeSecretKey(void) {
  ArrayResultByte r{nullptr, 0};
  guard([&] {
    Scheme& s = sch();
    REQUIRE(s.has_sk, "secret key not generated");
    std::vector<u64> h((size_t)(s.L + s.K) * s.N);
    download(h.data(), s.sR.p, h.size());
    Wire w; w.qp(h.data(), s.L, s.K, s.N);
    r = bytes_result(w.b);
    return 0;
  });
  return r;
}
int LoadSecretKey(const unsigned char* data, unsigned long len) {
  return guard([&] {
    Scheme& s = sch();
    const int N = s.N, nm = s.L + s.K;
    REQUIRE(data, "no data");
    std::vector<u64> h((size_t)nm * N);
    WireIn in{data, (size_t)len};
    in.qp(h.data(), s.L, s.K, N, s.mod, s.L);
    in.end();
    DU64 sR((size_t)nm * N); upload(sR.p, h.data(), h.size());
    // the ternary coefficients (for Galois keys) from limb q_0: out of Montgomery form, inverse NTT, centred
    DU64 c0((size_t)N); d2d(c0.p, sR.p, (size_t)N * 8);
    launch_mont_convert(c0.p, 0, 1, rows_q(0), s.d_mods.p, N, false, s.st);
    ntt(c0.p, 0, 1, rows_q(0), false);
    std::vector<u64> coef(N); download(coef.data(), c0.p, N);
    std::vector<int8_t> sv(N);
    const u64 q0 = s.mod[0];
    for (int x = 0; x < N; x++) {
      const u64 v = coef[x];
      REQUIRE(v <= 1 || v == q0 - 1, "secret key coefficients must be ternary");
      sv[x] = v == 0 ? 0 : (v == 1 ? 1 : -1);
    }
    sync();
    s.s = sv; s.sR = std::move(sR); s.has_sk = true;
    // keys derived from a previous secret are stale
    s.gkeys.clear(); s.rlk.reset(); s.seeded_gk.clear(); s.rlk_seeded = false;
    for (auto& kv : s.lts) kv.second->ptrs_ready = false;
    return 0;
  });
}
ArrayResultByte GenerateAndSerializeRotationKey(int galEl) {
  ArrayResultByte r{nullptr, 0};
  guard([&] {
    Scheme& s = sch();
    const u64 g = (u64)(unsigned)galEl;
    const bool had = s.gkeys.count(g) != 0;
    ensure_galois_key(g);
    r = bytes_result(serialize_galois_key(g, *s.gkeys.at(g)));
    if (!had) s.gkeys.erase(g);  // the reference returns the key without keeping it
    return 0;
  });
  return r;
}
int LoadRotationKey(const unsigned char* data, unsigned long len, unsigned long galEl) {
  return guard([&] {
    Scheme& s = sch();
    const int N = s.N, nm = s.L + s.K;
    REQUIRE(data, "no data");
    WireIn in{data, (size_t)len};
    REQUIRE(in.u64v() == (u64)galEl, "serialized key is for another Galois element");
    REQUIRE(in.u64v() == 2 * (u64)N, "serialized key is for another ring degree");
    REQUIRE(in.u64v() == 0, "base-two decomposition is not supported");
    REQUIRE(in.u64v() == (u64)s.dnum, "serialized key has another number of digits");
    std::vector<u64> h((size_t)s.dnum * 2 * nm * N);
    for (int d = 0; d < s.dnum; d++) {
      REQUIRE(in.u64v() == 1 && in.u64v() == 2, "malformed gadget ciphertext");
      for (int p = 0; p < 2; p++) in.qp(h.data() + ((size_t)d * 2 + p) * nm * N, s.L, s.K, N, s.mod, s.L);
    }
    in.end();
    auto k = std::make_unique<DU64>(h.size());
    upload(k->p, h.data(), h.size());
    s.gkeys[(u64)galEl] = std::move(k);
    s.seeded_gk.erase((u64)galEl);  // its a halves are read, not regenerated
    perm_for((u64)galEl); perm_inv_for((u64)galEl);
    s.lt_keys.insert((u64)galEl);
    // transforms cache key pointers: rebuild them on next use
    for (auto& kv : s.lts) kv.second->ptrs_ready = false;
    return 0;
  });
}
ArrayResultByte SerializeDiagonal(int transformID, int diagIdx) {
  ArrayResultByte r{nullptr, 0};
  guard([&] {
    Scheme& s = sch();
    LinTrans& t = get_lt(transformID);
    const int N = s.N, nqp = t.level + 1 + s.K;
    const int d = ((diagIdx % t.slots) + t.slots) % t.slots;
    auto it = std::find(t.plain_idx.begin(), t.plain_idx.end(), d);
    REQUIRE(it != t.plain_idx.end(), "diagonal not in the transform");
    const size_t p = it - t.plain_idx.begin();
    REQUIRE(t.resident[p], "diagonal not loaded");
    std::vector<u64> h((size_t)nqp * N);
    DU64 tmp((size_t)nqp * N);
    lt_diag_get(t, p, tmp.p);
    download(h.data(), tmp.p, h.size());
    Wire w; w.qp(h.data(), t.level + 1, s.K, N);
    r = bytes_result(w.b);
    // as the reference, the serialized diagonal leaves the transform
    t.resident[p] = 0;
    if (std::none_of(t.resident.begin(), t.resident.end(), [](char x) { return x != 0; })) t.diags.reset();
    return 0;
  });
  return r;
}
int LoadPlaintextDiagonal(const unsigned char* data, unsigned long len, int transformID, unsigned long diagIdx) {
  return guard([&] {
    Scheme& s = sch();
    LinTrans& t = get_lt(transformID);
    const int N = s.N, nqp = t.level + 1 + s.K, np = (int)t.plain_idx.size();
    REQUIRE(data, "no data");
    const int d = (int)(diagIdx % (unsigned long)t.slots);
    auto it = std::find(t.plain_idx.begin(), t.plain_idx.end(), d);
    REQUIRE(it != t.plain_idx.end(), "diagonal not in the transform");
    const size_t p = it - t.plain_idx.begin();
    std::vector<u64> h((size_t)nqp * N);
    WireIn in{data, (size_t)len};
    std::vector<u64> mods = qp_mods(t.level);
    in.poly(h.data(), t.level + 1, N, mods, 0);
    in.poly(h.data() + (size_t)(t.level + 1) * N, s.K, N, mods, t.level + 1);
    in.end();
    // storage was released with the last diagonal: np plaintexts + the all-zero one
    if (!t.diags.p) lt_alloc_diags(t, np);
    DU64 tmp((size_t)nqp * N);
    upload(tmp.p, h.data(), h.size());
    lt_diag_put(t, p, tmp.p);
    t.resident[p] = 1;
    return 0;
  });
}
// [ext] ciphertexts and plaintexts in the wire layout (no counterpart in the
// reference: its backends never serialize them)
ArrayResultByte SerializeCiphertext(int ciphertextID) {
  ArrayResultByte r{nullptr, 0};
  guard([&] {
    const Cipher& c = get_ct(ciphertextID);
    r = bytes_result(serialize_element(c.d.p, 2, c.level, c.scale, c.logslots));
    return 0;
  });
  return r;
}
int LoadCiphertext(const unsigned char* data, unsigned long len) {
  return guard([&] {
    int level, logslots;
    double scale;
    std::vector<u64> h = parse_element(data, (size_t)len, 2, level, scale, logslots);
    auto c = new_ct(level, scale);
    c->logslots = logslots;
    upload(c->d.p, h.data(), h.size());
    return push_ct(std::move(c));
  });
}
ArrayResultByte SerializePlaintext(int plaintextID) {
  ArrayResultByte r{nullptr, 0};
  guard([&] {
    const Plain& p = get_pt(plaintextID);
    r = bytes_result(serialize_element(p.d.p, 1, p.level, p.scale, p.logslots));
    return 0;
  });
  return r;
}
int LoadPlaintext(const unsigned char* data, unsigned long len) {
  return guard([&] {
    Scheme& s = sch();
    int level, logslots;
    double scale;
    std::vector<u64> h = parse_element(data, (size_t)len, 1, level, scale, logslots);
    auto p = std::make_unique<Plain>();
    p->level = level; p->scale = scale; p->logslots = logslots;
    p->d = DU64((size_t)(level + 1) * s.N);
    upload(p->d.p, h.data(), h.size());
    return push_pt(std::move(p));
  });
}
int RemovePlaintextDiagonals(int transformID) {
  return guard([&] {
    LinTrans& t = get_lt(transformID);
    sync();
    std::fill(t.resident.begin(), t.resident.end(), 0);
    t.diags.reset();
    return 0;
  });
}

// ---- tensors ----
int DeletePlaintext(int id) { return guard([&] { Scheme& s = sch(); if (s.pts.erase(id)) s.pt_ids.give(id); return 0; }); }
int DeleteCiphertext(int id) { return guard([&] { Scheme& s = sch(); if (s.cts.erase(id)) s.ct_ids.give(id); return 0; }); }
unsigned long GetPlaintextScale(int id) { unsigned long v = 0; guard([&] { v = scale_to_ulong(get_pt(id).scale); return 0; }); return v; }
unsigned long GetCiphertextScale(int id) { unsigned long v = 0; guard([&] { v = scale_to_ulong(get_ct(id).scale); return 0; }); return v; }
double GetCiphertextScaleDouble(int id) { double v = -1; guard([&] { v = get_ct(id).scale; return 0; }); return v; }
double GetPlaintextScaleDouble(int id) { double v = -1; guard([&] { v = get_pt(id).scale; return 0; }); return v; }
int SetPlaintextScale(int id, unsigned long scale) { return guard([&] { get_pt(id).scale = (double)scale; return 0; }); }
int SetCiphertextScale(int id, unsigned long scale) { return guard([&] { get_ct(id).scale = (double)scale; return 0; }); }
int GetPlaintextLevel(int id) { return guard([&] { return get_pt(id).level; }); }
int GetCiphertextLevel(int id) { return guard([&] { return get_ct(id).level; }); }
int GetPlaintextSlots(int id) { return guard([&] { return 1 << get_pt(id).logslots; }); }
int GetCiphertextSlots(int id) { return guard([&] { return 1 << get_ct(id).logslots; }); }
int GetCiphertextDegree(int id) { return guard([&] { get_ct(id); return 1; }); }
ArrayResultUInt64 GetModuliChain(void) {
  ArrayResultUInt64 r{nullptr, 0};
  guard([&] { Scheme& s = sch(); std::vector<u64> v(s.mod.begin(), s.mod.begin() + s.L); r.Data = (unsigned long long*)c_array(v); r.Length = v.size(); return 0; });
  return r;
}
ArrayResultUInt64 GetAuxModuliChain(void) {
  ArrayResultUInt64 r{nullptr, 0};
  guard([&] { Scheme& s = sch(); std::vector<u64> v(s.mod.begin() + s.L, s.mod.end()); r.Data = (unsigned long long*)c_array(v); r.Length = v.size(); return 0; });
  return r;
}
ArrayResultInt GetLivePlaintexts(void) {
  ArrayResultInt r{nullptr, 0};
  guard([&] { std::vector<int> v; for (auto& kv : sch().pts) v.push_back(kv.first); r.Data = c_array(v); r.Length = v.size(); return 0; });
  return r;
}
ArrayResultInt GetLiveCiphertexts(void) {
  ArrayResultInt r{nullptr, 0};
  guard([&] { std::vector<int> v; for (auto& kv : sch().cts) v.push_back(kv.first); r.Data = c_array(v); r.Length = v.size(); return 0; });
  return r;
}
void FreeCArray(void* ptr) { std::free(ptr); }

// ---- raw residue import/export (parity and measurement) ----
int ExportCiphertext(int id, uint64_t* buf, size_t len, int coeff) {
  return guard([&] {
    Scheme& s = sch(); Cipher& c = get_ct(id);
    size_t n = (size_t)2 * (c.level + 1) * s.N;
    REQUIRE(len >= n, "buffer too small");
    DU64 t(n); d2d(t.p, c.d.p, n * 8);
    if (coeff) ntt(t.p, (size_t)(c.level + 1) * s.N, 2, rows_q(c.level), false);
    download(buf, t.p, n);
    return (int)(n / s.N);
  });
}
int ImportCiphertext(const uint64_t* buf, int level, double scale, int coeff) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(level >= 0 && level < s.L, "invalid level");
    auto c = new_ct(level, scale);
    upload(c->d.p, buf, c->d.n);
    if (coeff) ntt(c->d.p, (size_t)(level + 1) * s.N, 2, rows_q(level), true);
    sync();
    return push_ct(std::move(c));
  });
}
int ExportPlaintext(int id, uint64_t* buf, size_t len, int coeff) {
  return guard([&] {
    Scheme& s = sch(); Plain& p = get_pt(id);
    size_t n = (size_t)(p.level + 1) * s.N;
    REQUIRE(len >= n, "buffer too small");
    DU64 t(n); d2d(t.p, p.d.p, n * 8);
    if (coeff) ntt(t.p, 0, 1, rows_q(p.level), false);
    download(buf, t.p, n);
    return (int)(n / s.N);
  });
}
int ImportPlaintext(const uint64_t* buf, int level, double scale, int coeff) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(level >= 0 && level < s.L, "invalid level");
    auto p = std::make_unique<Plain>();
    p->level = level; p->scale = scale; p->logslots = s.logN - 1; p->d = DU64((size_t)(level + 1) * s.N);
    upload(p->d.p, buf, p->d.n);
    if (coeff) ntt(p->d.p, 0, 1, rows_q(level), true);
    sync();
    return push_pt(std::move(p));
  });
}
int ExportGaloisKey(uint64_t galel, uint64_t* buf, size_t len) {
  return guard([&] {
    Scheme& s = sch();
    ensure_galois_key(galel);
    const DU64& k = *s.gkeys.at(galel);
    REQUIRE(len >= k.n, "buffer too small");
    DU64 t(k.n); d2d(t.p, k.p, k.bytes());
    launch_mont_convert(t.p, (size_t)(s.L + s.K) * s.N, 2 * s.dnum, rows_all(), s.d_mods.p, s.N, false, s.st);
    download(buf, t.p, k.n);
    return 0;
  });
}
int ExportSecretKey(int64_t* buf, size_t len) {
  return guard([&] { Scheme& s = sch(); REQUIRE(s.has_sk && len >= (size_t)s.N, "no secret key / buffer too small");
    for (int i = 0; i < s.N; i++) buf[i] = s.s[i]; return 0; });
}
int ExportLinearTransformDiagonal(int ltID, int diag, uint64_t* buf, size_t len) {
  return guard([&] {
    Scheme& s = sch(); LinTrans& t = get_lt(ltID);
    auto it = std::find(t.plain_idx.begin(), t.plain_idx.end(), diag);
    REQUIRE(it != t.plain_idx.end(), "diagonal not stored");
    size_t p = it - t.plain_idx.begin(), n = (size_t)(t.level + 1 + s.K) * s.N;
    REQUIRE(len >= n, "buffer too small");
    DU64 tmp(n); lt_diag_get(t, p, tmp.p);
    launch_mont_convert(tmp.p, 0, 1, RowMap{t.level + 1 + s.K, t.level + 1, 0, s.L, 0, 0}, s.d_mods.p, s.N, false, s.st);
    download(buf, tmp.p, n);
    return (int)(n / s.N);
  });
}
int GetLinearTransformInfo(int ltID, int* out, int len) {
  return guard([&] {
    LinTrans& t = get_lt(ltID);
    REQUIRE(len >= 4, "buffer too small");
    out[0] = t.N1; out[1] = (int)t.giant.size(); out[2] = (int)t.rot2.size(); out[3] = (int)t.plain_idx.size();
    return 0;
  });
}

int GetSchemeInfo(int* out, int len) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(len >= 6, "buffer too small");
    out[0] = s.logN; out[1] = s.L; out[2] = s.K; out[3] = s.dnum; out[4] = s.logscale; out[5] = s.h;
    return 0;
  });
}

// ---- device buffers owned by the library (callers without their own HIP runtime) ----
void* DeviceAlloc(size_t bytes) {
  void* p = nullptr;
  guard([&] {
    if (!g_pool) g_pool = new Pool();
    p = g_pool->get(bytes);
    g_pool->user_.insert(p);
    return 0;
  });
  return p;
}
// A buffer from DeviceAlloc is released by DeviceFree or by DeleteScheme
// (which releases all device memory): freeing it twice, or after the scheme
// was deleted, is an error.
int DeviceFree(void* ptr) {
  return guard([&] {
    REQUIRE(g_pool, "no device pool");
    if (!ptr) return 0;
    REQUIRE(g_pool->user_.count(ptr), "DeviceFree: not a live buffer from DeviceAlloc (freed twice, or released by DeleteScheme)");
    if (S) sync();
    g_pool->user_.erase(ptr);
    REQUIRE(g_pool->put(ptr), "DeviceFree: buffer is not live");
    return 0;
  });
}
int CopyToDevice(void* dst, const void* src, size_t bytes) {
  return guard([&] { HCHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); return 0; });
}
int CopyToHost(void* dst, const void* src, size_t bytes) {
  return guard([&] {
    if (S) sync();
    HCHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return 0;
  });
}

// ---- batched NTT and RNS multiply-accumulate on device buffers ----
int NttDevice(uint64_t* data, int npoly, int nrows, int forward) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(data && npoly > 0 && nrows > 0 && nrows <= s.L + s.K, "NttDevice: bad arguments");
    const RowMap rm{nrows, nrows, 0, 0, 0, 0};
    timed(forward ? "ntt_batch" : "intt_batch", [&] { ntt(data, (size_t)nrows * s.N, npoly, rm, forward != 0); });
    HCHECK(hipGetLastError());
    return 0;
  });
}
int MulAccDevice(const uint64_t* a, const uint64_t* b, uint64_t* out, int npoly, int nrows) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(a && b && out && npoly > 0 && nrows > 0 && nrows <= s.L + s.K, "MulAccDevice: bad arguments");
    timed("mulacc", [&] { launch_mulacc(a, b, out, npoly, nrows, s.d_mods.p, s.N, s.st); });
    HCHECK(hipGetLastError());
    return 0;
  });
}

// ---- stream / timing ----
int Synchronize(void) {
  return guard([&] {
    for (hipStream_t x : sch().streams)
      if (x) HCHECK(hipStreamSynchronize(x));
    return 0;
  });
}
int SetStream(int idx) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(idx == 0 || idx == 1, "stream index must be 0 or 1");
    if (!s.streams[idx]) HCHECK(hipStreamCreateWithFlags(&s.streams[idx], hipStreamNonBlocking));
    s.st = s.streams[idx];
    g_pool->cur = idx;
    return 0;
  });
}
int JoinStream(int idx) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(idx == 0 || idx == 1, "stream index must be 0 or 1");
    hipStream_t other = s.streams[idx];
    if (!other || other == s.st) return 0;
    if (!s.join_ev[idx]) HCHECK(hipEventCreateWithFlags(&s.join_ev[idx], hipEventDisableTiming));
    // the wait takes the event as recorded now; a later JoinStream records it anew
    HCHECK(hipEventRecord(s.join_ev[idx], other));
    HCHECK(hipStreamWaitEvent(s.st, s.join_ev[idx], 0));
    return 0;
  });
}
void* GetStream(void) { return S ? (void*)S->st : nullptr; }
// [ext] integer VALU issue rate, wave-instructions per second over the
// whole GPU: out[0] = the peak (the faster of the two probes), out[1] =
// compute units, out[2] = the peak per compute unit and clock at the
// device's peak clock, out[3] = v_mad_u64_u32 alone, out[4] = v_add3_u32.
int LaunchProbe(int limbs, double* out, int len) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(out && len >= 3, "LaunchProbe needs 3 outputs");
    REQUIRE(limbs >= 1 && limbs <= 256, "LaunchProbe: 1 to 256 limbs");
    const int reps = 200;
    const size_t words = (size_t)limbs * s.N;
    DU64 a(words), b(words), o(4096);
    HCHECK(hipMemsetAsync(a.p, 0, words * 8, s.st));
    HCHECK(hipMemsetAsync(b.p, 0, words * 8, s.st));
    hipEvent_t e0, e1;
    HCHECK(hipEventCreate(&e0)); HCHECK(hipEventCreate(&e1));
    auto time = [&](auto&& body) {
      for (int r = 0; r < reps; r++) body(r);  // warm-up
      HCHECK(hipEventRecord(e0, s.st));
      for (int r = 0; r < reps; r++) body(r);
      HCHECK(hipEventRecord(e1, s.st));
      HCHECK(hipEventSynchronize(e1));
      float ms = 0;
      HCHECK(hipEventElapsedTime(&ms, e0, e1));
      return (double)ms * 1e3 / reps;
    };
    out[0] = time([&](int r) { launch_empty_probe(o.p, 1024, r, s.st); });
    out[1] = time([&](int r) {
      if (r & 1) launch_copy(a.p, 0, b.p, 0, words, 1, s.st);
      else launch_copy(b.p, 0, a.p, 0, words, 1, s.st);
    });
    out[2] = 2.0 * words * 8 / (out[1] * 1e-6) / 1e12;
    (void)hipEventDestroy(e0); (void)hipEventDestroy(e1);
    return 0;
  });
}
int ValuPeakProbe(double* out, int len) {
  return guard([&] {
    Scheme& s = sch();
    REQUIRE(out && len >= 5, "ValuPeakProbe needs 5 outputs");
    int dev = 0;
    HCHECK(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    HCHECK(hipGetDeviceProperties(&prop, dev));
    const int cus = prop.multiProcessorCount, blocks = cus * 16, iters = 4096;
    DU64 buf((size_t)blocks * 256);
    hipEvent_t a, b;
    HCHECK(hipEventCreate(&a)); HCHECK(hipEventCreate(&b));
    double rate[2];
    for (int op = 0; op < 2; op++) {
      launch_valu_probe(op, buf.p, blocks, 3u, iters, s.st);  // warm-up (clocks up)
      HCHECK(hipEventRecord(a, s.st));
      launch_valu_probe(op, buf.p, blocks, 5u, iters, s.st);
      HCHECK(hipEventRecord(b, s.st));
      HCHECK(hipEventSynchronize(b));
      float ms = 0;
      HCHECK(hipEventElapsedTime(&ms, a, b));
      rate[op] = (double)blocks * (256 / 64) * iters * 8 / (ms * 1e-3);
    }
    (void)hipEventDestroy(a); (void)hipEventDestroy(b);
    out[0] = std::max(rate[0], rate[1]);
    out[1] = cus;
    out[2] = out[0] / cus / ((double)prop.clockRate * 1e3);
    out[3] = rate[0];
    out[4] = rate[1];
    return 0;
  });
}
int KernelTimingEnable(int on) { return guard([&] { Scheme& s = sch(); sync(); timing_collect(); s.timing.acc.clear(); s.timing.on = on != 0; return 0; }); }
int KernelTimingGet(const char* name, long* count, double* total_ms) {
  return guard([&] {
    Scheme& s = sch(); sync(); timing_collect();
    auto it = s.timing.acc.find(name);
    *count = it == s.timing.acc.end() ? 0 : it->second.first;
    *total_ms = it == s.timing.acc.end() ? 0.0 : it->second.second;
    return 0;
  });
}
// device-memory counterparts of the reference's Go heap sampler: the pool
// tracks every allocation, so the peak is exact rather than sampled
unsigned long long LiveHeapBytes(void) { return g_pool ? (unsigned long long)g_pool->live : 0ULL; }
int StartLiveHeapSampler(int intervalMs) {
  (void)intervalMs;
  return guard([&] { REQUIRE(g_pool, "no device pool"); sync(); g_pool->peak = g_pool->live; return 0; });
}
unsigned long long StopLiveHeapSampler(void) {
  unsigned long long v = 0;
  guard([&] { REQUIRE(g_pool, "no device pool"); sync(); v = g_pool->peak; return 0; });
  return v;
}
int GetMemoryStats(uint64_t* live, uint64_t* cached, uint64_t* peak) {
  return guard([&] { REQUIRE(g_pool, "no device pool"); *live = g_pool->live; *cached = g_pool->cached; *peak = g_pool->peak; return 0; });
}

}  // extern "C"
