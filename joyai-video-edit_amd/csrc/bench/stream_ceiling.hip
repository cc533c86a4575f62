// Bare row streams: the HBM ceiling of each row kernel's access shape.
//
// Measurement support only (bench.py loads it; the op library does not).
// A stream moves exactly the bytes of one row kernel, in the same launch
// shape, with none of its arithmetic: the same 256-thread workgroups, LPR
// lanes per row and CH 16-byte chunks per lane, the same nontemporal loads
// and 16- or 8-byte nontemporal stores, per-row fp32 scalars where the kernel
// writes scales, and the one dependency the algorithm imposes — no store of a
// row leaves before the whole row has arrived (a row norm or a row maximum
// needs all of it): every stored chunk folds in the XOR of all chunks of the
// lane, and rows that span several waves meet at a workgroup barrier, as the
// kernels' cross-wave reductions do.
//
// Row r of input stream t starts at in[t] + r * LPR*CH*16 bytes, row r of
// output stream o at out[o] + r * LPR*CH*OUTB bytes; with in[0] == out[0] and
// OUTB == 16 the stream is in place (the QK kernels' layout).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jo_device.hpp"

namespace {

using jo::u32x2;
using jo::u32x4;

struct StreamArgs {
  const char* in[3];
  char* out[2];
  float* scal;       // nscal fp32 per row, or null
  int64_t rows;
  int nscal;
  uint32_t mask;     // 0 at run time; keeps the dependency opaque to the compiler
};

template <int LPR, int CH, int NIN, int NOUT, int OUTB>
__global__ __launch_bounds__(256) void stream_rows_kernel(const StreamArgs a) {
  constexpr int RPB = 256 / LPR;
  constexpr int64_t kIn = int64_t(LPR) * CH * 16;
  constexpr int64_t kOut = int64_t(LPR) * CH * OUTB;
  const int lane = threadIdx.x % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const bool ok = row < a.rows;
  u32x4 c[NIN][CH];
#pragma unroll
  for (int t = 0; t < NIN; ++t)
#pragma unroll
    for (int i = 0; i < CH; ++i)
      c[t][i] = ok ? jo::ld16_nt(a.in[t] + row * kIn + (i * LPR + lane) * 16)
                   : u32x4{0u, 0u, 0u, 0u};
  uint32_t x = 0;
#pragma unroll
  for (int t = 0; t < NIN; ++t)
#pragma unroll
    for (int i = 0; i < CH; ++i) x ^= c[t][i].x ^ c[t][i].y ^ c[t][i].z ^ c[t][i].w;
  uint32_t dep = x & a.mask;
  if constexpr (LPR > jo::kWave) dep = __syncthreads_or(dep) ? a.mask : 0u;
  if (!ok) return;
#pragma unroll
  for (int o = 0; o < NOUT; ++o) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const u32x4 v = c[o % NIN][i];
      if constexpr (OUTB == 16)
        jo::st16_nt(a.out[o] + row * kOut + (i * LPR + lane) * 16,
                    u32x4{v.x ^ dep, v.y ^ dep, v.z ^ dep, v.w ^ dep});
      else
        jo::st8_nt(a.out[o] + row * kOut + (i * LPR + lane) * 8,
                   u32x2{v.x ^ v.y ^ dep, v.z ^ v.w ^ dep});
    }
  }
  if (a.scal && lane < a.nscal) a.scal[row * a.nscal + lane] = static_cast<float>(x & 0xffu);
}

template <int LPR, int CH, int NIN, int NOUT, int OUTB>
bool try_launch(int lpr, int ch, int nin, int nout, int outb, const StreamArgs& a,
                hipStream_t st) {
  if (lpr != LPR || ch != CH || nin != NIN || nout != NOUT || outb != OUTB) return false;
  constexpr int RPB = 256 / LPR;
  hipLaunchKernelGGL((stream_rows_kernel<LPR, CH, NIN, NOUT, OUTB>),
                     dim3(static_cast<unsigned>((a.rows + RPB - 1) / RPB)), dim3(256), 0, st, a);
  return true;
}

}  // namespace

// Shapes measured by bench.py: (lanes per row, chunks per lane, input
// streams, output streams, bytes stored per 16 bytes read). Returns 0 on
// success, 1 for a shape that is not instantiated, 3 for a launch error.
extern "C" int jo_stream_rows(const void* in0, const void* in1, const void* in2, void* out0,
                              void* out1, float* scal, int64_t rows, int lpr, int ch, int nin,
                              int nout, int outb, int nscal, void* stream) {
  if (rows <= 0 || rows > (int64_t{1} << 30)) return 1;
  StreamArgs a{{static_cast<const char*>(in0), static_cast<const char*>(in1),
                static_cast<const char*>(in2)},
               {static_cast<char*>(out0), static_cast<char*>(out1)},
               scal, rows, nscal, 0u};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool done =
      // QK units: 1, 2 or 3 head groups of 512 elements per wave, in place or to a cache
      try_launch<64, 1, 1, 1, 16>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<64, 2, 1, 1, 16>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<64, 3, 1, 1, 16>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<64, 4, 1, 1, 16>(lpr, ch, nin, nout, outb, a, st) ||
      // bf16 rows -> fp8 rows (+ scales): hidden 3072 / 4096 / 16384
      try_launch<64, 6, 1, 1, 8>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<128, 3, 1, 1, 8>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<256, 2, 1, 1, 8>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<128, 4, 1, 1, 8>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<64, 8, 1, 1, 8>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<256, 8, 1, 1, 8>(lpr, ch, nin, nout, outb, a, st) ||
      // two rows in, two rows out (residual add + norm): hidden 3072
      try_launch<128, 3, 2, 2, 16>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<64, 6, 2, 2, 16>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<256, 2, 2, 2, 16>(lpr, ch, nin, nout, outb, a, st) ||
      // three rows in (x, scale, shift), one out: hidden 4096
      try_launch<256, 2, 3, 1, 16>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<64, 8, 3, 1, 16>(lpr, ch, nin, nout, outb, a, st) ||
      // one row in, one out, 16 bytes each: rmsnorm rows of 128 and 4096
      try_launch<16, 1, 1, 1, 16>(lpr, ch, nin, nout, outb, a, st) ||
      try_launch<64, 8, 1, 1, 16>(lpr, ch, nin, nout, outb, a, st);
  if (!done) return 1;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}
