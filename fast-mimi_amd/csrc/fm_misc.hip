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

// Up to two byte buffers copied in one launch: 16-byte vectors where the
// pointers allow, bytes otherwise.
struct CopyPair {
  const unsigned char* src[2];
  unsigned char* dst[2];
  long bytes[2];
  long vec[2];  // 16-byte vectors copied as such (the rest byte by byte)
};

__global__ __launch_bounds__(256) void copy_buffers_kernel(CopyPair a) {
  const long stride = (long)gridDim.x * 256, first = (long)blockIdx.x * 256 + threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint4* s = reinterpret_cast<const uint4*>(a.src[i]);
    uint4* d = reinterpret_cast<uint4*>(a.dst[i]);
    for (long e = first; e < a.vec[i]; e += stride) d[e] = s[e];
    for (long e = a.vec[i] * 16 + first; e < a.bytes[i]; e += stride) a.dst[i][e] = a.src[i][e];
  }
}

}  // namespace

extern "C" {

int fm_copy_buffers(const void* src0, void* dst0, size_t bytes0, const void* src1, void* dst1,
                    size_t bytes1, hipStream_t stream) {
  if ((bytes0 && (!src0 || !dst0)) || (bytes1 && (!src1 || !dst1))) return FM_BAD_ARGUMENT;
  if ((long)bytes0 < 0 || (long)bytes1 < 0) return FM_BAD_ARGUMENT;
  CopyPair a{};
  const void* src[2] = {src0, src1};
  void* dst[2] = {dst0, dst1};
  const size_t bytes[2] = {bytes0, bytes1};
  long most = 0;
  for (int i = 0; i < 2; ++i) {
    a.src[i] = static_cast<const unsigned char*>(src[i]);
    a.dst[i] = static_cast<unsigned char*>(dst[i]);
    a.bytes[i] = bytes[i] ? (long)bytes[i] : 0;
    const bool aligned = ((reinterpret_cast<uintptr_t>(src[i]) | reinterpret_cast<uintptr_t>(dst[i])) & 15) == 0;
    a.vec[i] = aligned ? a.bytes[i] / 16 : 0;
    const long work = a.vec[i] + (a.bytes[i] - 16 * a.vec[i]);
    most = work > most ? work : most;
  }
  if (most == 0) return FM_OK;
  const long blocks = (most + 255) / 256;
  hipLaunchKernelGGL(copy_buffers_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0,
                     stream, a);
  return (int)hipGetLastError();
}

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
