// Small memory-bound kernels of the Mimi hot path and library identity.

#include "fm_common.h"

namespace {

// Depthwise causal ConvTranspose1d (groups == channels), trimmed to L*stride:
// y[b, q*s + r, c] = sum_{j} x[b, q - j, c] * w[c, r + j*s],  j = 0..k/s-1, q-j >= 0.
// The sum runs j = taps-1 .. 0 (earliest input first), each product rounded.
__global__ __launch_bounds__(256) void upsample_depthwise_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ w,
                                                                 int B, int L, int C, int k, int s,
                                                                 float* __restrict__ y) {
  const long total = (long)B * L * s * C;
  const int taps = k / s;
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < total; e += (long)gridDim.x * 256) {
    const int c = (int)(e % C);
    const long o = e / C;  // output position within all batches
    const long b = o / ((long)L * s);
    const int tout = (int)(o - b * (long)L * s);
    const int q = tout / s, r = tout - q * s;
    float acc = 0.0f;
    bool first = true;
    for (int j = taps - 1; j >= 0; --j) {
      const int qi = q - j;
      if (qi < 0) continue;
      const float prod = __fmul_rn(x[(b * L + qi) * C + c], w[(long)c * k + r + j * s]);
      acc = first ? prod : __fadd_rn(acc, prod);
      first = false;
    }
    y[e] = acc;
  }
}

}  // namespace

extern "C" {

int fm_upsample_depthwise(const float* x, int batch, int length, int channels,
                          const float* weight, int kernel, int stride, float* y,
                          hipStream_t stream) {
  if (!x || !weight || !y || batch < 0 || length < 0 || channels <= 0 || stride <= 0 ||
      kernel <= 0 || kernel % stride)
    return FM_BAD_ARGUMENT;
  const long total = (long)batch * length * stride * channels;
  if (total == 0) return FM_OK;
  const long blocks = (total + 255) / 256;
  hipLaunchKernelGGL(upsample_depthwise_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                     dim3(256), 0, stream, x, weight, batch, length, channels, kernel, stride, y);
  return (int)hipGetLastError();
}

// ABI version of this library (bumped when an entry point's contract changes).
int fm_abi_version(void) { return 1; }

}  // extern "C"
