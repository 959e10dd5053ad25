// encoder.hip -- CKKS encoding on the device (Lattigo ckks.Encoder algorithm).
//
// A plaintext of `slots` = N/2 real values becomes N integer coefficients:
//   1. the values (fp32 as they cross the ABI, widened to float64) go through
//      the special inverse FFT over the rotation group 5^j mod 2N (DIF
//      butterflies len = slots .. 2, then bit reversal and division by slots);
//   2. real parts are coefficients [0, slots), imaginary parts [slots, N),
//      each scaled and rounded to a fixed-point integer (|v|*scale + 0.5
//      truncated below 2^64, exact mantissa * 2^e above);
//   3. the integer is reduced into every row of the plaintext's RNS basis.
// The forward NTT and the Montgomery conversion that follow are the library's
// own kernels.
//
// Every floating-point operation is the one of the host restatement, in the
// same order, with contraction into fused multiply-adds switched off, so the
// coefficients are bit-identical to a scalar float64 evaluation of the
// algorithm.  One thread per butterfly and one launch per FFT stage: encoding
// is set-up work (diagonals are encoded once per compiled layer) and a stage
// launch over a batch of plaintexts streams at HBM rate.
#include "hipckks.h"
#include "kernels.h"

namespace {

// plaintext p, element k: data[src * slots + ((k + rot) mod slots)], or 0 past
// nvals; complex input: (re, im) pairs at data[2k], data[2k + 1]
__global__ void encode_load_kernel(double* __restrict__ re, double* __restrict__ im, size_t pstride,
                                   const float* __restrict__ data, const EncodeSrc* __restrict__ src, int n, int nvals,
                                   int complex_in) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  const int p = blockIdx.y;
  if (k >= n) return;
  const EncodeSrc e = src[p];
  double v = 0.0, vi = 0.0;
  if (k < nvals) {
    if (complex_in) {
      v = (double)data[2 * (size_t)k];
      vi = (double)data[2 * (size_t)k + 1];
    } else {
      v = (double)data[(size_t)e.src * n + ((k + e.rot) & (n - 1))];
    }
  }
  re[(size_t)p * pstride + k] = v;
  im[(size_t)p * pstride + k] = vi;
}

// one DIF stage of the special inverse FFT: blocks of len, pairs (k, k + len/2)
__global__ void special_ifft_stage_kernel(double* __restrict__ re, double* __restrict__ im, size_t pstride, int n, int len,
                                          int M, const int* __restrict__ rotgroup, const double* __restrict__ rre,
                                          const double* __restrict__ rim) {
#pragma clang fp contract(off)
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (n >> 1)) return;
  double* R = re + (size_t)blockIdx.y * pstride;
  double* I = im + (size_t)blockIdx.y * pstride;
  const int lenh = len >> 1, lenq = len << 2, gap = M / lenq, mask = lenq - 1;
  const int j = t % lenh;
  const int k = (t / lenh) * len + j;
  const double ur = R[k], ui = I[k], vr = R[k + lenh], vi = I[k + lenh];
  const int idx = (lenq - (rotgroup[j] & mask)) * gap;
  const double wr = rre[idx], wi = rim[idx];
  const double dr = ur - vr, di = ui - vi;
  R[k] = ur + vr;
  I[k] = ui + vi;
  R[k + lenh] = dr * wr - di * wi;
  I[k + lenh] = dr * wi + di * wr;
}

// fixed-point record of one coefficient (Lattigo SingleFloat64ToFixedPointCRT)
__device__ __forceinline__ void fixed_point(double value, double scale, u64& mag, u64& meta) {
#pragma clang fp contract(off)
  if (value == 0) { mag = 0; meta = 0; return; }
  u64 neg = 0;
  if (value < 0) { neg = 1; scale *= -1; }
  value *= scale;
  if (value >= 1.8446744073709552e+19) {
    int e;
    const double m = frexp(value, &e);
    mag = (u64)ldexp(m, 53);
    meta = neg | ((u64)(e - 53) << 8);
  } else {
    mag = (u64)(value + 0.5);
    meta = neg;
  }
}

__device__ __forceinline__ int brv_bits(int x, int bits) { return (int)(__brev((unsigned)x) >> (32 - bits)); }

// coefficient x of plaintext p: bit reversal, division by n, fixed point, residues in every row of rm
__global__ void encode_finish_kernel(u64* __restrict__ out, size_t out_pstride, RowMap rm, const double* __restrict__ re,
                                     const double* __restrict__ im, size_t pstride, int n, int logn, double scale,
                                     const ModC* __restrict__ mods, int N) {
#pragma clang fp contract(off)
  const int x = blockIdx.x * blockDim.x + threadIdx.x;
  if (x >= N) return;
  const int p = blockIdx.y;
  const int i = x < n ? x : x - n;
  const int k = brv_bits(i, logn);
  const double v = (x < n ? re : im)[(size_t)p * pstride + k] / (double)n;
  u64 mag, meta;
  fixed_point(v, scale, mag, meta);
  const int neg = (int)(meta & 1), ex = (int)(meta >> 8);
  u64* o = out + (size_t)p * out_pstride;
  for (int a = 0; a < rm.nact(); a++) {
    const int row = rm.row(a);
    const ModC mc = mods[rm.mod(row)];
    u64 r = mont_mul(mag, mc.rmod, mc.q, mc.qinv);  // mag mod q
    for (int e = 0; e < ex; e++) r = add_mod(r, r, mc.q);
    if (neg && r) r = mc.q - r;
    o[(size_t)row * N + x] = r;
  }
}

}  // namespace

void launch_encode_fft(u64* out, size_t out_pstride, RowMap rm, const float* data, const EncodeSrc* src, int np, int nvals,
                       double scale, double* re, double* im, size_t pstride, const int* rotgroup, const double* rre,
                       const double* rim, const ModC* mods, int logN, hipStream_t st, bool complex_in) {
  const int N = 1 << logN, n = N >> 1, M = 2 * N, logn = logN - 1;
  const int tpb = 256;
  hipLaunchKernelGGL(encode_load_kernel, dim3((n + tpb - 1) / tpb, np), dim3(tpb), 0, st, re, im, pstride, data, src, n, nvals,
                     complex_in ? 1 : 0);
  for (int len = n; len >= 2; len >>= 1)
    hipLaunchKernelGGL(special_ifft_stage_kernel, dim3((n / 2 + tpb - 1) / tpb, np), dim3(tpb), 0, st, re, im, pstride, n, len,
                       M, rotgroup, rre, rim);
  hipLaunchKernelGGL(encode_finish_kernel, dim3((N + tpb - 1) / tpb, np), dim3(tpb), 0, st, out, out_pstride, rm, re, im,
                     pstride, n, logn, scale, mods, N);
}
