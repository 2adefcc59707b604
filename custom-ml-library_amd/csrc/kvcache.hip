// KV-cache append into the reference's int8 format (src/tensorsmith/nn/
// cache.py:54-86, quantiser at :73-77): for every appended row x = src[b, h,
// t, 0:D] (already in the cache dtype), in fp32,
//   s = max(max_d |x_d| / 127, 1e-8),   q_d = round_half_even(x_d / s),
// stored as int8 at dst[b, h, pos + t, d] with s at scale[b, h, pos + t].
// One kernel does the reduction, the division, the rounding and both writes,
// so an append is one pass over the new rows.  Division is IEEE (correctly
// rounded) and rint rounds half to even, as NumPy's round does: the stored
// bytes and scales are bit-identical to the reference's.
#include "mfma_common.h"

namespace tsattn {
namespace {

constexpr int NT = 256;

template <typename T>
__global__ __launch_bounds__(NT) void kv_append_int8_kernel(int B, int H, int T_, int D, View src,
                                                            View dst, View scale, int64_t pos) {
  // one wave per row (b, h, t); lane handles elements lane, lane + 64, ...
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (NT / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= static_cast<int64_t>(B) * H * T_) return;
  const int t = static_cast<int>(row % T_);
  const int64_t bh = row / T_;
  const int h = static_cast<int>(bh % H), b = static_cast<int>(bh / H);
  const T *x = static_cast<const T *>(src.data) + b * src.s0 + h * src.s1 + static_cast<int64_t>(t) * src.s2;
  int8_t *q = static_cast<int8_t *>(const_cast<void *>(dst.data)) + b * dst.s0 + h * dst.s1 +
              (pos + t) * dst.s2;
  constexpr int PER = 8;  // D <= 512
  float v[PER];
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int d = lane + 64 * j;
    v[j] = d < D ? static_cast<float>(x[d]) : 0.f;
    m = fmaxf(m, fabsf(v[j]));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  const float s = fmaxf(m / 127.f, 1e-8f);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int d = lane + 64 * j;
    if (d < D) q[d] = static_cast<int8_t>(rintf(v[j] / s));
  }
  if (lane == 0)
    static_cast<float *>(const_cast<void *>(scale.data))[b * scale.s0 + h * scale.s1 + (pos + t) * scale.s2] = s;
}

}  // namespace

hipError_t launch_kv_append_int8(int dtype, int B, int H, int T_, int D, View src, View dst,
                                 View scale, int64_t pos, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(B) * H * T_;
  const dim3 grid(static_cast<unsigned>((rows + NT / 64 - 1) / (NT / 64))), block(NT);
  Probe pr_("kv_append_int8", st);
  if (dtype == TSATTN_F32) kv_append_int8_kernel<float><<<grid, block, 0, st>>>(B, H, T_, D, src, dst, scale, pos);
  else if (dtype == TSATTN_F16) kv_append_int8_kernel<f16><<<grid, block, 0, st>>>(B, H, T_, D, src, dst, scale, pos);
  else kv_append_int8_kernel<bf16><<<grid, block, 0, st>>>(B, H, T_, D, src, dst, scale, pos);
  return hipGetLastError();
}

}  // namespace tsattn
