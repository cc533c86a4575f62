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
// Row r of input stream t starts at in[t] + r * LPR*CH*16 bytes (or, for
// input rows that come in groups of G contiguous rows GS bytes apart — the
// per-head rows of a strided [T, H, D] view — at in[t] + (r / G) * GS +
// (r % G) * LPR*CH*16), row r of output stream o at out[o] + r * LPR*CH*OUTB
// bytes; with in[0] == out[0] and OUTB == 16 the stream is in place (the QK
// kernels' layout). NCONST row-invariant inputs (a weight or modulation row
// every row uses, read through the cache by every row as the kernels do)
// follow the row inputs in in[]; OUT8 adds an output stream of 8 bytes per 16
// read (an fp8 row next to a bf16 one) after the NOUT outputs in out[].
// flags bit 0 (wt): the 16-byte row stores use the system-scope nontemporal
// policy (jo::st16_sys_nt), as the in-place QK kernels' row stores do; bit 1
// (xcd): workgroups take their row blocks in jo::xcd_row_block order, as the
// per-token quantizer does.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jo_device.hpp"

namespace {

using jo::u32x2;
using jo::u32x4;

struct StreamArgs {
  const char* in[5];
  char* out[3];
  float* scal;       // nscal fp32 per row, or null
  int64_t rows;
  uint32_t group_rows;    // input rows per contiguous group (0: all rows contiguous)
  int64_t group_stride;   // bytes between groups
  int nscal;
  int wt;            // 16-byte row stores written through (sc0 sc1 nt)
  int xcd;           // row blocks in xcd_row_block order
  uint32_t mask;     // 0 at run time; keeps the dependency opaque to the compiler
};

template <int LPR, int CH, int NIN, int NOUT, int OUTB, int NCONST, int OUT8>
__global__ __launch_bounds__(256) void stream_rows_kernel(const StreamArgs a) {
  static_assert(NIN + NCONST <= 5 && NOUT + OUT8 <= 3, "stream counts");
  constexpr int RPB = 256 / LPR;
  constexpr int64_t kIn = int64_t(LPR) * CH * 16;
  constexpr int64_t kOut = int64_t(LPR) * CH * OUTB;
  const int lane = threadIdx.x % LPR;
  const int64_t blk = a.xcd ? jo::xcd_row_block<RPB>(blockIdx.x, gridDim.x) : blockIdx.x;
  const int64_t row = blk * RPB + threadIdx.x / LPR;
  const bool ok = row < a.rows;
  u32x4 w[NCONST > 0 ? NCONST : 1][CH];
#pragma unroll
  for (int t = 0; t < NCONST; ++t)
#pragma unroll
    for (int i = 0; i < CH; ++i) w[t][i] = jo::ld16(a.in[NIN + t] + (i * LPR + lane) * 16);
  int64_t ro = row * kIn;
  if (a.group_rows) {
    const uint32_t g = static_cast<uint32_t>(row) / a.group_rows;
    ro = static_cast<int64_t>(g) * a.group_stride + (row - int64_t{g} * a.group_rows) * kIn;
  }
  u32x4 c[NIN][CH];
#pragma unroll
  for (int t = 0; t < NIN; ++t)
#pragma unroll
    for (int i = 0; i < CH; ++i)
      c[t][i] = ok ? jo::ld16_nt(a.in[t] + ro + (i * LPR + lane) * 16) : u32x4{0u, 0u, 0u, 0u};
  uint32_t x = 0;
#pragma unroll
  for (int t = 0; t < NCONST; ++t)
#pragma unroll
    for (int i = 0; i < CH; ++i) x ^= w[t][i].x ^ w[t][i].y ^ w[t][i].z ^ w[t][i].w;
#pragma unroll
  for (int t = 0; t < NIN; ++t)
#pragma unroll
    for (int i = 0; i < CH; ++i) x ^= c[t][i].x ^ c[t][i].y ^ c[t][i].z ^ c[t][i].w;
  uint32_t dep = x & a.mask;
  if constexpr (LPR > jo::kWave) {
    // The rows' waves meet once, through LDS, as the kernels' cross-wave
    // reductions do: each wave's lane 0 posts its part, one barrier, and every
    // wave reads the parts of its row.
    __shared__ uint32_t part[256 / jo::kWave];
    const int wave = threadIdx.x / jo::kWave;
    dep = __ballot(dep != 0u) ? a.mask : 0u;
    if ((threadIdx.x & (jo::kWave - 1)) == 0) part[wave] = dep;
    __syncthreads();
    constexpr int kWpr = LPR / jo::kWave;
    const int first = (wave / kWpr) * kWpr;
    dep = 0u;
#pragma unroll
    for (int k = 0; k < kWpr; ++k) dep |= part[first + k];
  }
  if (!ok) return;
#pragma unroll
  for (int o = 0; o < NOUT; ++o) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const u32x4 v = c[o % NIN][i];
      if constexpr (OUTB == 16) {
        const u32x4 sv{v.x ^ dep, v.y ^ dep, v.z ^ dep, v.w ^ dep};
        if (a.wt) {
          // the wave's first row as the (wave-uniform) base of the resource
          const int64_t row0 = __builtin_amdgcn_readfirstlane(static_cast<int>(row));
          jo::st16_sys_nt(a.out[o] + row0 * kOut,
                          static_cast<int>((row - row0) * kOut + (i * LPR + lane) * 16), sv);
        } else {
          jo::st16_nt(a.out[o] + row * kOut + (i * LPR + lane) * 16, sv);
        }
      } else
        jo::st8_nt(a.out[o] + row * kOut + (i * LPR + lane) * 8,
                   u32x2{v.x ^ v.y ^ dep, v.z ^ v.w ^ dep});
    }
  }
  if constexpr (OUT8) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const u32x4 v = c[NIN - 1][i];
      jo::st8_nt(a.out[NOUT] + row * (kIn / 2) + (i * LPR + lane) * 8,
                 u32x2{v.x ^ v.z ^ dep, v.y ^ v.w ^ dep});
    }
  }
  if (a.scal && lane < a.nscal) a.scal[row * a.nscal + lane] = static_cast<float>(x & 0xffu);
}

template <int LPR, int CH, int NIN, int NOUT, int OUTB, int NCONST = 0, int OUT8 = 0>
bool try_launch(int lpr, int ch, int nin, int nout, int outb, int nconst, int out8,
                const StreamArgs& a, hipStream_t st) {
  if (lpr != LPR || ch != CH || nin != NIN || nout != NOUT || outb != OUTB || nconst != NCONST ||
      out8 != OUT8)
    return false;
  constexpr int RPB = 256 / LPR;
  hipLaunchKernelGGL((stream_rows_kernel<LPR, CH, NIN, NOUT, OUTB, NCONST, OUT8>),
                     dim3(static_cast<unsigned>((a.rows + RPB - 1) / RPB)), dim3(256), 0, st, a);
  return true;
}

}  // namespace

// Shapes measured by bench.py: (lanes per row, chunks per lane, row input
// streams, output streams, bytes stored per 16 bytes read, row-invariant
// inputs, extra 8-byte output). in[] holds nin + nconst pointers, out[]
// nout + out8; flags as StreamArgs.wt (bit 0) and .xcd (bit 1). Returns 0 on
// success, 1 for a shape that is not instantiated or bad sizes, 3 for a
// launch error.
extern "C" int jo_stream_rows(const void* const* in, void* const* out, float* scal, int64_t rows,
                              int lpr, int ch, int nin, int nout, int outb, int nscal, int nconst,
                              int out8, int64_t group_rows, int64_t group_stride, int flags,
                              void* stream) {
  if (rows <= 0 || rows > (int64_t{1} << 30)) return 1;
  if (group_rows < 0 || group_rows > (int64_t{1} << 30) || (group_rows && group_stride <= 0))
    return 1;
  if (nin < 1 || nconst < 0 || nin + nconst > 5 || nout < 0 || out8 < 0 || out8 > 1 ||
      nout + out8 > 3 || !in || !out)
    return 1;
  if (nscal < 0 || nscal > 64 || (nscal > 0 && !scal)) return 1;
  StreamArgs a{};
  for (int t = 0; t < nin + nconst; ++t) {
    if (!in[t]) return 1;
    a.in[t] = static_cast<const char*>(in[t]);
  }
  for (int o = 0; o < nout + out8; ++o) {
    if (!out[o]) return 1;
    a.out[o] = static_cast<char*>(out[o]);
  }
  a.scal = scal;
  a.rows = rows;
  a.group_rows = static_cast<uint32_t>(group_rows);
  a.group_stride = group_stride;
  a.nscal = nscal;
  if (flags & ~3) return 1;
  a.wt = flags & 1;
  a.xcd = (flags >> 1) & 1;
  a.mask = 0u;
  hipStream_t st = static_cast<hipStream_t>(stream);
#define TRY(...) try_launch<__VA_ARGS__>(lpr, ch, nin, nout, outb, nconst, out8, a, st)
  const bool done =
      // QK units: 1, 2 or 3 head groups of 512 elements per wave, in place or to a cache
      TRY(64, 1, 1, 1, 16) ||
      TRY(64, 2, 1, 1, 16) ||
      TRY(64, 2, 1, 1, 16, 0, 1) ||   // QK pass that also writes the pre-RoPE K stage
      TRY(64, 3, 1, 1, 16) ||
      TRY(64, 4, 1, 1, 16) ||
      // bf16 rows -> fp8 rows (+ scales): hidden 3072 / 4096 / 16384
      TRY(64, 6, 1, 1, 8) ||
      TRY(128, 3, 1, 1, 8) ||
      TRY(256, 2, 1, 1, 8) ||
      TRY(128, 4, 1, 1, 8) ||
      TRY(64, 8, 1, 1, 8) ||
      TRY(256, 8, 1, 1, 8) ||
      // two rows in, two rows out (residual add + norm): hidden 3072, with
      // the broadcast scale and shift rows, and the FP8 epilogue's shape
      // (residual out, fp8 row out, gate / scale / shift rows)
      TRY(128, 3, 2, 2, 16) ||
      TRY(128, 3, 2, 2, 16, 2) ||
      TRY(128, 3, 2, 1, 16, 3, 1) ||
      TRY(64, 6, 2, 2, 16) ||
      TRY(256, 2, 2, 2, 16) ||
      // three rows in (x, scale, shift), one out: hidden 4096
      TRY(256, 2, 3, 1, 16) ||
      TRY(64, 8, 3, 1, 16) ||
      // one row in, one out, 16 bytes each: rmsnorm rows of 128 and 4096
      TRY(16, 1, 1, 1, 16) ||
      TRY(64, 8, 1, 1, 16) ||
      // the same with the row-invariant weight row the kernels read per row
      TRY(64, 6, 1, 1, 8, 1) ||    // RMSNorm -> FP8, hidden 3072
      TRY(128, 3, 1, 1, 8, 1) ||   // the same rows, two waves per row
      TRY(16, 1, 1, 1, 16, 1) ||   // rmsnorm rows of 128 (also per-head rows of a strided view)
      TRY(64, 8, 1, 1, 16, 1);     // rmsnorm rows of 4096
#undef TRY
  if (!done) return 1;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}
