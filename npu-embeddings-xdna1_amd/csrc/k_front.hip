// k_front.hip -- the HBM-bound pieces of the ViT and Whisper front ends and
// the ViT head (the GEMMs themselves run on the encoder GEMM):
//   vit_patches_k    pixels [B, 3, H, W] fp32 -> bf16 patch rows [B*np, 3*p*p]
//                    in (c, ky, kx) order, the Conv2d weight order
//                    (vit/encoder.cpp:288-332 consumes these rows);
//   vit_assemble_k   x = [cls; patch rows] + positions (vit/encoder.cpp:
//                    309-329: CLS prepended, then every row + its position);
//   gather_rows_bf16_k  rows r*stride of an fp32 matrix -> bf16 [n, d] (the
//                    ViT CLS rows for the head, head.cpp:16-49);
//   mel_time_major_k mel [B, mels, T] fp32 -> bf16 [B, T+2, mels] with a zero
//                    row before and after each sample: row t+1 holds frame t,
//                    so the three taps of a k=3, pad-1 convolution at frame t
//                    are rows t, t+1, t+2 -- one contiguous run of 3*mels
//                    values (whisper/features.cpp:390-469).
#include "mx_common.hpp"
#include "mx_kernels.hpp"

using namespace mxd;

namespace {

// One thread per 8 consecutive values of a patch row (8 | p).
__global__ __launch_bounds__(256) void vit_patches_k(const float *__restrict__ px, int64_t B,
                                                     int img, int p, uint16_t *__restrict__ rows) {
  const int gp = img / p, np = gp * gp, pd = 3 * p * p, per_row = pd / 8;
  const int64_t total = B * np * per_row;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row;
    const int k = (int)(i - r * per_row) * 8;
    const int64_t b = r / np;
    const int pi = (int)(r - b * np), py = pi / gp, pxi = pi - py * gp;
    const int c = k / (p * p), rem = k - c * p * p, ky = rem / p, kx = rem - ky * p;
    const float *src = px + ((b * 3 + c) * (int64_t)img + (py * p + ky)) * img + pxi * p + kx;
    const float4 a = *(const float4 *)src, d = *(const float4 *)(src + 4);
    uint4 o;
    o.x = pack_bf2(a.x, a.y);
    o.y = pack_bf2(a.z, a.w);
    o.z = pack_bf2(d.x, d.y);
    o.w = pack_bf2(d.z, d.w);
    *(uint4 *)(rows + r * pd + k) = o;
  }
}

// x[b*(np+1)] = cls + pos[0]; x[b*(np+1) + 1 + i] = patch[b*np + i] + pos[1 + i].
__global__ __launch_bounds__(256) void vit_assemble_k(const float *__restrict__ patch,
                                                      const float *__restrict__ cls,
                                                      const float *__restrict__ pos, int64_t B,
                                                      int np, int d, float *__restrict__ x) {
  const int d4 = d / 4;
  const int64_t total = B * (np + 1) * d4;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / d4;
    const int c = (int)(i - row * d4) * 4;
    const int64_t b = row / (np + 1);
    const int t = (int)(row - b * (np + 1));
    const float4 src = t == 0 ? *(const float4 *)(cls + c)
                              : *(const float4 *)(patch + (b * np + t - 1) * d + c);
    const float4 pe = *(const float4 *)(pos + (int64_t)t * d + c);
    *(float4 *)(x + row * d + c) =
        make_float4(src.x + pe.x, src.y + pe.y, src.z + pe.z, src.w + pe.w);
  }
}

__global__ __launch_bounds__(256) void gather_rows_bf16_k(const float *__restrict__ x,
                                                          int64_t stride, int64_t n, int d,
                                                          uint16_t *__restrict__ out) {
  const int d4 = d / 4;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n * d4;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / d4;
    const int c = (int)(i - r * d4) * 4;
    const float4 v = *(const float4 *)(x + r * stride + c);
    *(uint2 *)(out + r * d + c) = make_uint2(pack_bf2(v.x, v.y), pack_bf2(v.z, v.w));
  }
}

// One thread per (sample, padded row, mel); rows 0 and T+1 are zero.
__global__ __launch_bounds__(256) void mel_time_major_k(const float *__restrict__ mel, int64_t B,
                                                        int mels, int T,
                                                        uint16_t *__restrict__ out) {
  const int64_t total = B * (int64_t)(T + 2) * mels;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / mels;
    const int m = (int)(i - row * mels);
    const int64_t b = row / (T + 2);
    const int t = (int)(row - b * (T + 2)) - 1;
    out[i] = (t >= 0 && t < T) ? f2bf(mel[(b * mels + m) * (int64_t)T + t]) : (uint16_t)0;
  }
}

inline int grid_of(int64_t items) {
  int64_t g = (items + 255) / 256;
  return (int)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

}  // namespace

namespace mxk {

hipError_t vit_patches(const float *px, int64_t B, int img, int p, uint16_t *rows,
                       hipStream_t s) {
  const int64_t items = B * (int64_t)(img / p) * (img / p) * (3 * p * p / 8);
  vit_patches_k<<<grid_of(items), 256, 0, s>>>(px, B, img, p, rows);
  return hipGetLastError();
}

hipError_t vit_assemble(const float *patch, const float *cls, const float *pos, int64_t B,
                        int np, int d, float *x, hipStream_t s) {
  vit_assemble_k<<<grid_of(B * (np + 1) * (d / 4)), 256, 0, s>>>(patch, cls, pos, B, np, d, x);
  return hipGetLastError();
}

hipError_t gather_rows_bf16(const float *x, int64_t stride, int64_t n, int d, uint16_t *out,
                            hipStream_t s) {
  gather_rows_bf16_k<<<grid_of(n * (d / 4)), 256, 0, s>>>(x, stride, n, d, out);
  return hipGetLastError();
}

hipError_t mel_time_major(const float *mel, int64_t B, int mels, int T, uint16_t *out,
                          hipStream_t s) {
  mel_time_major_k<<<grid_of(B * (int64_t)(T + 2) * mels), 256, 0, s>>>(mel, B, mels, T, out);
  return hipGetLastError();
}

}  // namespace mxk
