// The dropout keep mask of an attention problem, materialised: the mask the
// MFMA kernels regenerate on the fly (philox.h), written out as bytes so it
// can be inspected and checked against numpy.random.Philox on the host.
// One thread per 16-word block of a query row.
#include "philox.h"

namespace tsattn {
namespace {

constexpr int NT = 256;

__global__ __launch_bounds__(NT) void dropout_keep_kernel(Problem p, uint8_t *out) {
  const int bpr = (p.Sk + 15) / 16;  // blocks per row
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (idx >= rows * bpr) return;
  const int64_t row = idx / bpr;
  const int j16 = static_cast<int>(idx - row * bpr) * 16;
  uint64_t w[4];
  dropout_block(p.drop, dropout_block_index(p, row, j16), w);
  uint8_t *o = out + row * p.Sk + j16;
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const uint32_t word = static_cast<uint32_t>(w[m >> 2] >> (16 * (m & 3))) & 0xFFFFu;
    if (j16 + m < p.Sk) o[m] = p.drop.on ? (word >= p.drop.thr ? 1 : 0) : 1;
  }
}

}  // namespace

hipError_t launch_dropout_keep(const Problem &p, uint8_t *out, hipStream_t st) {
  const int64_t threads = static_cast<int64_t>(p.B) * p.Hq * p.Sq * ((p.Sk + 15) / 16);
  Probe pr_("dropout_keep", st);
  dropout_keep_kernel<<<dim3(static_cast<unsigned>((threads + NT - 1) / NT)), NT, 0, st>>>(p, out);
  return hipGetLastError();
}

}  // namespace tsattn
