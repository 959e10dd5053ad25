/*
 * helrm_hip.h -- C ABI of the MI355X (gfx950) CKKS backend for the HE-LRM
 * embedding PCMM (libhelrm_hip.so, built from helrm_amd/csrc/).
 *
 * The entry points keep the names, argument meaning, handle semantics and
 * return conventions of the cgo exports of Orion's Lattigo backend
 * (reference: the Go files of orion/backend/lattigo, bound by ctypes in
 * orion/backend/lattigo/bindings.py), so a ctypes binding written for that
 * library binds this one.  Differences, all deliberate:
 *   - functions that return void in the Lattigo library return int here:
 *     0 on success, -1 on failure; handle-returning functions return -1 on
 *     failure.  The message is available from GetLastError().  (Lattigo
 *     panics and aborts the process instead.)
 *   - array results use the same {Data, Length} structs, malloc'ed by the
 *     library and released with FreeCArray.
 * Entry points marked [ext] have no counterpart in the reference; they exist
 * for parity checks (explicit moduli, seeds and raw residues) and for
 * measurement.
 */
#ifndef HELRM_HIP_H
#define HELRM_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* orion/backend/lattigo/bindings.py:801-815 (ArrayResult* ctypes structs) */
typedef struct { int* Data; unsigned long Length; } ArrayResultInt;
typedef struct { float* Data; unsigned long Length; } ArrayResultFloat;
typedef struct { unsigned long long* Data; unsigned long long Length; } ArrayResultUInt64;
typedef struct { char* Data; unsigned long Length; } ArrayResultByte;

/* ---- scheme --------------------------------------------------------------- */
/* orion/backend/lattigo/scheme.go:34-87 NewScheme (primes generated from the
 * bit sizes as rlwe.GenModuli; keysPath/ioMode accepted, unused). */
int NewScheme(int logN, int* logQ, int lenQ, int* logP, int lenP, int logScale,
              int h, const char* ringType, const char* keysPath, const char* ioMode);
/* orion/backend/lattigo/scheme.go:88-100 DeleteScheme */
int DeleteScheme(void);
/* [ext] scheme from explicit moduli and a key/randomness seed */
int NewSchemeWithModuli(int logN, const uint64_t* q, int lenQ, const uint64_t* p,
                        int lenP, int logScale, int h, uint64_t seed);
/* [ext] seed used by the next NewScheme (default: /dev/urandom) */
void SetSchemeSeed(uint64_t seed);
/* [ext] the prime chain NewScheme would use */
int GeneratePrimes(int logN, const int* logQ, int lenQ, const int* logP, int lenP,
                   uint64_t* q, uint64_t* p);
/* [ext] last error message of the calling thread */
const char* GetLastError(void);

/* ---- key generator ---------------------------------------------------------- */
int NewKeyGenerator(void);            /* keygenerator.go:12 */
int GenerateSecretKey(void);          /* keygenerator.go:17 */
int GeneratePublicKey(void);          /* keygenerator.go:22 */
int GenerateRelinearizationKey(void); /* keygenerator.go:27-30 (evaluation key s^2 -> s) */
int GenerateEvaluationKeys(void);     /* keygenerator.go:32 */
/* Serialization for Orion's io_mode save/load (key_generator.py:17-31).  Byte
 * layout: this library's own, modelled on the structure of Lattigo v6's
 * WriteTo (row counts, lengths, then little-endian u64 words; see runtime.hip
 * "binary wire format").  Byte equality with Lattigo's MarshalBinary is not
 * established (no Lattigo here to compare with).  Results are released with
 * FreeCArray. */
ArrayResultByte SerializeSecretKey(void);                        /* keygenerator.go:38-47 */
int LoadSecretKey(const unsigned char* data, unsigned long len); /* keygenerator.go:49-58 */

/* ---- encoder ------------------------------------------------------------------ */
int NewEncoder(void);                                                      /* encoder.go:10 */
int Encode(const float* values, int lenValues, int level, unsigned long scale); /* encoder.go:15-30 */
ArrayResultFloat Decode(int plaintextID);                                  /* encoder.go:32-47 */
int DecodeDouble(int plaintextID, double* out, int len);                   /* [ext] Decode before the float cast */
int EncodeComplex(const float* values, int lenValues, int level, unsigned long scale); /* encoder.go:50-70 ((re, im) pairs) */
ArrayResultFloat DecodeComplex(int plaintextID);                           /* encoder.go:72-91 (interleaved re, im) */

/* ---- encryptor -------------------------------------------------------------- */
int NewEncryptor(void);              /* encryptor.go:9 */
int NewDecryptor(void);              /* encryptor.go:14 */
int Encrypt(int plaintextID);        /* encryptor.go:19-27 */
int Decrypt(int ciphertextID);       /* encryptor.go:29-38 */
int SetEncryptionCounter(uint64_t v); /* [ext] index of the next encryption's randomness */
/* Seeded ("compressed") upload of the Cheddar bindings: secret-key encryption
 * whose `a` is expanded from `seed` on the device (a[i][x] = uniform draw
 * rand64(seed, i*N + x) mod q_i in the NTT domain), so only b and the seed
 * cross the wire; DropAx zeroes a, ExpandSeededAx rebuilds it in place. */
int EncryptSeeded(int plaintextID, unsigned long long seed);   /* cheddar_pybind.cu:638-647 */
int DropAx(int ciphertextID);                                  /* cheddar_pybind.cu:650-655 (returns 0) */
int ExpandSeededAx(int ciphertextID, unsigned long long seed); /* cheddar_pybind.cu:657-660 (returns 0) */
double GetCiphertextBytes(int ciphertextID);                   /* cheddar_pybind.cu:666-673 */
double GetCiphertextBxBytes(int ciphertextID);                 /* cheddar_pybind.cu:676-679 */

/* ---- evaluator ---------------------------------------------------------------- */
int NewEvaluator(void);                   /* evaluator.go:13-35 (+ power-of-two and conjugation keys) */
int AddRotationKey(int rotation);         /* evaluator.go:37-52 */
int Rotate(int ciphertextID, int amount); /* evaluator.go:80-87 */
int RotateNew(int ciphertextID, int amount); /* evaluator.go:89-101 */
/* [ext] ciphertextID <- ciphertextID + Rotate(ciphertextID, amount), one step
 * of a Linear's output fold (`out += out.roll(k)`, linear.py:115-117 ->
 * RotateNew evaluator.go:89-101 + AddCiphertext evaluator.go:297-304) with
 * the add done in the key switch's last pass.  Same words as RotateNew +
 * AddCiphertext.  Returns ciphertextID. */
int RotateAdd(int ciphertextID, int amount);
/* [ext] No counterpart in the reference.  For callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops): RotateNew
 * written into the existing ciphertext outID (!= ciphertextID, with room for
 * the input's level), calling no hipMalloc / hipFree.  The key switch's
 * temporaries live in a static 96 MiB device array per GPU (a rotation at
 * N = 2^16 with up to 24 Q and 8 P limbs fits; larger levels are refused
 * with an error); the rotation key must already exist.  A call on the
 * scheme's other stream waits for the previous call's key switch before it
 * uses the array; calls from several host threads or processes on one GPU
 * race on it.  Returns outID. */
int RotateInto(int ciphertextID, int amount, int outID);
int Conjugate(int ciphertextID);          /* evaluator.go:103-114 */
int ConjugateNew(int ciphertextID);       /* evaluator.go:116-128 */
int Rescale(int ciphertextID);            /* evaluator.go:130-136 */
int RescaleNew(int ciphertextID);         /* evaluator.go:138-146 (rescales the input in place too) */
int AddPlaintext(int ciphertextID, int plaintextID);     /* evaluator.go:228-235 */
int AddPlaintextNew(int ciphertextID, int plaintextID);  /* evaluator.go:237-249 */
int SubPlaintext(int ciphertextID, int plaintextID);     /* evaluator.go:251-258 */
int SubPlaintextNew(int ciphertextID, int plaintextID);  /* evaluator.go:260-272 */
int AddCiphertext(int ctID0, int ctID1);                 /* evaluator.go:297-304 */
int AddCiphertextNew(int ctID0, int ctID1);              /* evaluator.go:306-318 */
int SubCiphertext(int ctID0, int ctID1);                 /* evaluator.go:320-327 */
int SubCiphertextNew(int ctID0, int ctID1);              /* evaluator.go:329-341 */
int Negate(int ciphertextID);                            /* evaluator.go:68-78 (Mul by -1.0: a new ciphertext) */
int MulImaginaryUnitNew(int ciphertextID); /* cheddar_pybind.cu:1827-1833 (times i = X^(N/2), key-free) */
int MulImaginaryUnit(int ciphertextID);    /* cheddar_pybind.cu:1834-1840 (in place) */
int AddScalar(int ciphertextID, float scalar);           /* evaluator.go:148-154 (round(scalar * scale) into part 0) */
int AddScalarNew(int ciphertextID, float scalar);        /* evaluator.go:156-166 */
int SubScalar(int ciphertextID, float scalar);           /* evaluator.go:168-174 */
int SubScalarNew(int ciphertextID, float scalar);        /* evaluator.go:176-186 */
int MulScalarInt(int ciphertextID, int scalar);          /* evaluator.go:188-194 (scale unchanged) */
int MulScalarIntNew(int ciphertextID, int scalar);       /* evaluator.go:196-206 */
int MulScalarFloat(int ciphertextID, float scalar);      /* evaluator.go:208-214 (non-integer: round(scalar * q_l), scale x q_l) */
int MulScalarFloatNew(int ciphertextID, float scalar);   /* evaluator.go:216-226 */
int MulPlaintext(int ciphertextID, int plaintextID);     /* evaluator.go:274-281 (level min, scales multiply, no rescale) */
int MulPlaintextNew(int ciphertextID, int plaintextID);  /* evaluator.go:283-295 */
int MulRelinCiphertext(int ctID0, int ctID1);            /* evaluator.go:343-350 (tensor + relinearize, no rescale) */
int MulRelinCiphertextNew(int ctID0, int ctID1);         /* evaluator.go:352-364 */

/* ---- polynomial evaluator (polyeval.go) ------------------------------------------ */
int NewPolynomialEvaluator(void);                                   /* polyeval.go:32-35 */
int GenerateMonomial(const float* coeffs, int lenCoeffs);           /* polyeval.go:37-47 (lowest degree first) */
int GenerateChebyshev(const float* coeffs, int lenCoeffs);          /* polyeval.go:49-60 (degree <= 3, on [-1, 1]) */
/* polyeval.go:62-84: a new ciphertext at scale outScale; degree <= 3 at depth
 * ceil(log2(degree + 1)) (orion/nn/activation.py:22-28). */
int EvaluatePolynomial(int ctInID, int polyID, unsigned long outScale);

/* ---- linear transforms -------------------------------------------------------- */
int NewLinearTransformEvaluator(void);   /* lineartransform.go:30-34 */
/* lineartransform.go:36-93 (diagonals as C floats, LevelQ = level,
 * Scale = Q[level], LogBabyStepGiantStepRatio = int(ln(bsgsRatio))). */
int GenerateLinearTransform(const int* diagIdxs, int diagIdxsLen, const float* diagData,
                            int diagDataLen, int level, float bsgsRatio, const char* ioMode);
int EvaluateLinearTransform(int transformID, int ctxtID);         /* lineartransform.go:95-113 */
/* [ext] on != 0: EvaluateLinearTransform returns Rescale(result) (the
 * lt_output_prerescaled convention of cheddar/bindings.py:183-187, read by
 * lt_evaluator.py:262-273), the first division fused into the final ModDown,
 * residues identical to EvaluateLinearTransform followed by Rescale.  Per
 * scheme, default 0.  Get returns the current setting (0 without a scheme). */
int SetLinearTransformPrerescale(int on);
int GetLinearTransformPrerescale(void);
ArrayResultInt GetLinearTransformRotationKeys(int transformID);   /* lineartransform.go:115-122 */
int GenerateLinearTransformRotationKey(int galEl);                /* lineartransform.go:124-128 */
int DeleteLinearTransform(int id);                                /* lineartransform.go:25-28 */
int RemoveRotationKeys(void);                                     /* lineartransform.go:203-211 */
/* io_mode save / load of rotation keys and diagonals (lt_evaluator.py:133-161, 440-497) */
ArrayResultByte GenerateAndSerializeRotationKey(int galEl);       /* lineartransform.go:130-140 (key not kept) */
int LoadRotationKey(const unsigned char* data, unsigned long len, unsigned long galEl); /* lineartransform.go:142-160 */
ArrayResultByte SerializeDiagonal(int transformID, int diagIdx);  /* lineartransform.go:162-177 (diagonal leaves the transform) */
int LoadPlaintextDiagonal(const unsigned char* data, unsigned long len, int transformID,
                          unsigned long diagIdx);                 /* lineartransform.go:179-193 */
int RemovePlaintextDiagonals(int transformID);                    /* lineartransform.go:195-201 */
/* [ext] ciphertexts and plaintexts in this library's wire layout: a header of
 * its own (scale as float64 bits, log2 slots, flags, count), then the vector
 * of ring.Poly in the NTT domain with standard representatives.  The header
 * is not Lattigo's MetaData encoding and byte parity with Lattigo is
 * unpinned.  No counterpart in the reference, whose backends never serialize
 * them; they carry the objects of a cross-check bundle (inputs and expected
 * outputs) that a machine with Lattigo would convert. */
ArrayResultByte SerializeCiphertext(int ciphertextID);
int LoadCiphertext(const unsigned char* data, unsigned long len);   /* returns a new ciphertext id */
ArrayResultByte SerializePlaintext(int plaintextID);
int LoadPlaintext(const unsigned char* data, unsigned long len);    /* returns a new plaintext id */

/* ---- tensors -------------------------------------------------------------------- */
int DeletePlaintext(int plaintextID);                       /* tensors.go:34-37 */
int DeleteCiphertext(int ciphertextID);                     /* tensors.go:39-42 */
unsigned long GetPlaintextScale(int plaintextID);           /* tensors.go:44-50 (UINT64_MAX above 2^64) */
unsigned long GetCiphertextScale(int ciphertextID);         /* tensors.go:52-58 */
int SetPlaintextScale(int plaintextID, unsigned long scale); /* tensors.go:60-64 */
int SetCiphertextScale(int ciphertextID, unsigned long scale); /* tensors.go:66-70 */
int GetPlaintextLevel(int plaintextID);                     /* tensors.go:72-76 */
int GetCiphertextLevel(int ciphertextID);                   /* tensors.go:78-82 */
int GetPlaintextSlots(int plaintextID);                     /* tensors.go:84-89 */
int GetCiphertextSlots(int ciphertextID);                   /* tensors.go:91-96 */
int GetCiphertextDegree(int ciphertextID);                  /* tensors.go:98-102 */
ArrayResultUInt64 GetModuliChain(void);                     /* tensors.go:104-109 */
ArrayResultUInt64 GetAuxModuliChain(void);                  /* tensors.go:111-116 */
ArrayResultInt GetLivePlaintexts(void);                     /* tensors.go:118-123 */
ArrayResultInt GetLiveCiphertexts(void);                    /* tensors.go:125-130 */
void FreeCArray(void* ptr);                                 /* utils.go:96-99 */
double GetCiphertextScaleDouble(int ciphertextID);          /* [ext] scale as a double (no 2^64 clamp) */
double GetPlaintextScaleDouble(int plaintextID);            /* [ext] */

/* ---- [ext] raw residues (limb-major u64[rows][N]; coeff != 0: coefficient
 *      domain, else the NTT domain; standard representatives in [0, q)) ---- */
int ExportCiphertext(int ciphertextID, uint64_t* buf, size_t len, int coeff);
int ImportCiphertext(const uint64_t* buf, int level, double scale, int coeff);
int ExportPlaintext(int plaintextID, uint64_t* buf, size_t len, int coeff);
int ImportPlaintext(const uint64_t* buf, int level, double scale, int coeff);
int ExportGaloisKey(uint64_t galEl, uint64_t* buf, size_t len); /* [dnum][2][L+K][N], NTT */
int ExportSecretKey(int64_t* buf, size_t len);                   /* ternary coefficients */
int ExportLinearTransformDiagonal(int transformID, int diag, uint64_t* buf, size_t len);
int GetLinearTransformInfo(int transformID, int* out, int len);  /* N1, giant, baby, plaintexts */
int GetSchemeInfo(int* out, int len);  /* logN, L, K, dnum, logScale, h */

/* ---- [ext] device buffers from the library's allocator (for callers that have
 *      no HIP runtime of their own; one process should use one HIP runtime) ---- */
void* DeviceAlloc(size_t bytes);                           /* NULL on failure */
/* -1 for a pointer freed twice or released by DeleteScheme.  Pointers carry
 * no owner: a stale pointer whose address a later DeviceAlloc returned again
 * frees that newer buffer. */
int DeviceFree(void* ptr);
int CopyToDevice(void* dst, const void* src, size_t bytes);  /* synchronous */
int CopyToHost(void* dst, const void* src, size_t bytes);    /* waits for the scheme stream first */

/* ---- [ext] batched transforms on device buffers (kernel microbenchmark) ----------
 * `data`, `a`, `b`, `out` are device pointers to npoly polynomials of nrows limbs
 * (limb-major u64[npoly][nrows][N], canonical residues; limb r uses modulus r
 * of the chain q_0..q_{L-1}, p_0..).  Work is queued on the scheme stream;
 * Synchronize() waits for it. */
int NttDevice(uint64_t* data, int npoly, int nrows, int forward);  /* in place; forward != 0: NTT, else inverse */
int MulAccDevice(const uint64_t* a, const uint64_t* b, uint64_t* out, int npoly, int nrows); /* out = sum_p a_p*b_p */

/* ---- [ext] stream and measurement ------------------------------------------------ */
int Synchronize(void);                                            /* waits for both streams */
void* GetStream(void);                                            /* hipStream_t the scheme's calls run on now */
/* [ext] two HIP streams per scheme, for independent chains of calls (no
 * counterpart in the reference, whose forward is one sequence).  SetStream(i)
 * makes stream i (0 or 1; 1 is created on first use, default priority) the
 * one every later call is ordered on; JoinStream(i) makes the current stream
 * wait for all work given to stream i so far.  Device buffers freed while
 * stream i is current are reused only by stream i: free an object while the
 * stream that last used it is current, or after joining that stream. */
int SetStream(int idx);
int JoinStream(int idx);
/* [ext] integer VALU issue-rate probe (measurement only), wave-instructions
 * per second over the GPU: out[0] = peak (the faster probe), out[1] = compute
 * units, out[2] = the peak per compute unit per clock (peak clock), out[3] =
 * v_mad_u64_u32 alone, out[4] = v_add3_u32 alone. */
int ValuPeakProbe(double* out, int len);
/* [ext] launch-latency probe (measurement only), HIP events over 200
 * dependent launches on the current stream: out[0] = microseconds per launch
 * of an empty kernel of 1,024 workgroups, out[1] = microseconds per copy of
 * `limbs` rows of N words (read and written), out[2] = that copy's TB/s. */
int LaunchProbe(int limbs, double* out, int len);
int KernelTimingEnable(int on);                                   /* HIP events around named launches */
int KernelTimingGet(const char* name, long* count, double* total_ms);
int GetMemoryStats(uint64_t* live, uint64_t* cached, uint64_t* peak);
/* memstats.go:40-86: device-memory bytes held by the library's allocator (the
 * reference samples the Go heap); the peak between Start and Stop is exact */
unsigned long long LiveHeapBytes(void);
int StartLiveHeapSampler(int intervalMs);
unsigned long long StopLiveHeapSampler(void);

#ifdef __cplusplus
}
#endif
#endif
