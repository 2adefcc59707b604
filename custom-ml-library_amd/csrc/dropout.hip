// The dropout keep mask of an attention problem, materialised: as bytes (one
// thread per 16-word group of a query row), so it can be inspected and
// checked against the host's restatement of the stream, and as the bits the
// MFMA backward reads (philox.h draws the words).
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

// The keep bits (DropDesc::bits layout), one thread per 32-bit word: the
// word of row i and keys 32 t .. + 31 from two 16-word blocks.  Padding rows
// (i >= Sq) and keys past Sk hold zeros.
__global__ __launch_bounds__(NT) void dropout_bits_kernel(Problem p, uint32_t *out) {
  const DropDesc &d = p.drop;
  const int64_t words = static_cast<int64_t>(p.B) * p.Hq * d.nkt * d.sqp;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (idx >= words) return;
  const int64_t line = idx / d.sqp;  // (b Hq + h) nkt + t
  const int i = static_cast<int>(idx - line * d.sqp);
  const int64_t bh = line / d.nkt;
  const int t = static_cast<int>(line - bh * d.nkt);
  uint32_t bits = 0;
  if (i < p.Sq) {
    const int64_t row = bh * p.Sq + i;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int j16 = 32 * t + 16 * half;
      if (j16 >= p.Sk) break;
      uint64_t w[4];
      dropout_block(d, dropout_block_index(p, row, j16), w);
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const uint32_t word = static_cast<uint32_t>(w[m >> 2] >> (16 * (m & 3))) & 0xFFFFu;
        if (j16 + m < p.Sk && word >= d.thr) bits |= 1u << (16 * half + m);
      }
    }
  }
  out[idx] = bits;
}

}  // namespace

hipError_t launch_dropout_bits(const Problem &p, uint32_t *out, hipStream_t st) {
  const int64_t words = static_cast<int64_t>(p.B) * p.Hq * p.drop.nkt * p.drop.sqp;
  Probe pr_("dropout_bits", st);
  dropout_bits_kernel<<<dim3(static_cast<unsigned>((words + NT - 1) / NT)), NT, 0, st>>>(p, out);
  return hipGetLastError();
}

hipError_t launch_dropout_keep(const Problem &p, uint8_t *out, hipStream_t st) {
  const int64_t threads = static_cast<int64_t>(p.B) * p.Hq * p.Sq * ((p.Sk + 15) / 16);
  Probe pr_("dropout_keep", st);
  dropout_keep_kernel<<<dim3(static_cast<unsigned>((threads + NT - 1) / NT)), NT, 0, st>>>(p, out);
  return hipGetLastError();
}

}  // namespace tsattn
