// Row-wise scaled FP8 GEMM with bias (drop-in for the reference's
// fp8_scaled_mm, deploy/joyomni_ops/csrc/fp8_gemm.cu:1450-1546):
//   out[m, n] = round_out( scale_a[m] * (acc[m, n] * scale_b[n]) + bias[n] ),
//   acc[m, n] = sum_k A[m, k] * B[k, n]   (fp8 e4m3fn operands, fp32 accumulate)
// with A [M, K] row-major and B [K, N] column-major (each column's K bytes
// contiguous, i.e. B^T [N, K] row-major) — the epilogue order of the
// reference's visitor tree (fp8_gemm.cu:99-136: acc * scale_b, then
// scale_a * that + bias, round to nearest).
//
// gfx950 design: one 256-thread workgroup per 256x256 output tile; the four
// waves own 128x128 quadrants computed with v_mfma_f32_32x32x64_f8f6f4
// (4x4 MFMA tiles, 256 fp32 accumulators per lane). K advances in 128-byte
// stages: every thread loads 8 sixteen-byte chunks of A and 8 of B^T from
// HBM into registers for the next stage while the MFMAs run on the current
// one, then writes them to the other half of a double-buffered LDS tile
// (2 x 64 KB). LDS rows are 128 bytes; chunk c of row r is stored at chunk
// position c ^ (r % 8) ^ ((r / 8) % 2), so the 16 rows a 16-lane group
// reads with one ds_read_b128 fall in 16 distinct 16-byte bank groups.

#include <atomic>
#include <type_traits>

#include "jo_device.hpp"
#include "jo_host.hpp"

namespace jo {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 128;                      // bytes of K per stage
constexpr int kStageBytes = (kBM + kBN) * kBK;  // A tile then B tile
constexpr int kChunksPerThread = kBM * kBK / 16 / kBlock;  // 8 (same for B)

struct GemmArgs {
  const uint8_t* a;  // [M, K], row stride lda (bytes)
  const uint8_t* b;  // B^T [N, K], row stride ldb (bytes)
  const float* sa;   // [M]
  const float* sb;   // [N]
  const void* bias;  // [N] out dtype, optional
  void* out;         // [M, N] out dtype, row stride ldo (elements)
  int64_t lda, ldb, ldo;
  int M, N, K;
  float* ws = nullptr;  // split K: fp32 partial products [splits, M, N]
};

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// One 32x32x64 fp8 MFMA with unit block scales (lowered to the unscaled
// v_mfma_f32_32x32x64_f8f6f4).
__device__ __forceinline__ f32x16 mfma32(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

template <class OutTag>
__global__ __launch_bounds__(kBlock, 1) void fp8_gemm_kernel(const GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStageBytes];  // 2 stages
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

  // Global chunk q = tid + 256 j of a 256 x 128-byte tile: row q / 8, chunk q % 8.
  // Rows beyond M (N) read row M-1 (N-1): their results are never stored.
  // Chunks beyond K read as zero so they add nothing.
  const uint8_t* ga[kChunksPerThread];
  const uint8_t* gb[kChunksPerThread];
  int lds_off[kChunksPerThread];
#pragma unroll
  for (int j = 0; j < kChunksPerThread; ++j) {
    const int q = tid + kBlock * j;
    const int r = q >> 3, c = q & 7;
    const int ra = min(m0 + r, g.M - 1), rb = min(n0 + r, g.N - 1);
    ga[j] = g.a + static_cast<int64_t>(ra) * g.lda + c * 16;
    gb[j] = g.b + static_cast<int64_t>(rb) * g.ldb + c * 16;
    lds_off[j] = r * kBK + ((c ^ swz(r)) << 4);
  }
  const int stages = (g.K + kBK - 1) / kBK;
  u32x4 ra[kChunksPerThread], rb[kChunksPerThread];
  auto load_stage = [&](int s) {
    const int kb = s * kBK;
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
      const int c = (tid + kBlock * j) & 7;
      const bool in_k = kb + c * 16 < g.K;
      ra[j] = in_k ? ld16(ga[j] + kb) : u32x4{0u, 0u, 0u, 0u};
      rb[j] = in_k ? ld16(gb[j] + kb) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_stage = [&](int buf) {
    uint8_t* base = smem + buf * kStageBytes;
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
      *reinterpret_cast<u32x4*>(base + lds_off[j]) = ra[j];
      *reinterpret_cast<u32x4*>(base + kBM * kBK + lds_off[j]) = rb[j];
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment read offsets: tile row (l % 32) of subtile i, chunk pair
  // (l / 32) * 2 + {0, 1} of k-slice s (4 chunks per 64-byte slice).
  const int fr = lane & 31, fh = lane >> 5;

  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int s = 0; s < stages; ++s) {
    const int buf = s & 1;
    if (s + 1 < stages) load_stage(s + 1);
    const uint8_t* As = smem + buf * kStageBytes;
    const uint8_t* Bs = As + kBM * kBK;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      i32x8 af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wm * 128 + i * 32 + fr;
        const int c = ks * 4 + fh * 2;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(As + r * kBK + ((c ^ swz(r)) << 4));
        const u32x4 hi = *reinterpret_cast<const u32x4*>(As + r * kBK + (((c + 1) ^ swz(r)) << 4));
        af[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = wn * 128 + j * 32 + fr;
        const int c = ks * 4 + fh * 2;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(Bs + r * kBK + ((c ^ swz(r)) << 4));
        const u32x4 hi = *reinterpret_cast<const u32x4*>(Bs + r * kBK + (((c + 1) ^ swz(r)) << 4));
        bf[j] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(af[i], bf[j], acc[i][j]);
    }
    if (s + 1 < stages) store_stage(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds column n = n0 + wn*128 + j*32 + (l % 32) of subtile
  // (i, j), rows m = m0 + wm*128 + i*32 + (e / 4)*8 + (l / 32)*4 + e % 4.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 128 + j * 32 + fr;
    if (n >= g.N) continue;
    const float sbn = g.sb[n];
    const float bn = g.bias ? load_elem<OutTag>(g.bias, n) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * 128 + i * 32 + (e >> 2) * 8 + fh * 4 + (e & 3);
        if (m < g.M) {
          const float t = acc[i][j][e] * sbn;
          store_elem<OutTag>(g.out, static_cast<int64_t>(m) * g.ldo + n, __builtin_fmaf(g.sa[m], t, bn));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Pipelined kernel (K % 64 == 0): NW waves on a BM x BN tile (BM 256 or 224),
// in a 2 x NW/2 grid of wave tiles 128 (or 96, the second row of a 224-row
// tile) x 2*BN/NW (NW = 8: two waves per SIMD, so one wave's barrier and LDS
// waits overlap the other's MFMAs). K advances in 64-byte stages through a
// ring of NST LDS stages of (BM + BN) x 64 bytes filled by direct
// global->LDS loads issued NST stages ahead, and each wave holds the
// next stage's fragments in a second register set while the current stage's
// MFMAs run. LDS rows are 64 bytes; chunk c of row r sits at chunk position
// c ^ ((r >> 2) & 3). gfx950's LDS serves a ds_read_b128 sixteen lanes per
// cycle from 64 four-byte banks: the sixteen consecutive rows a 16-lane group
// reads then fall in sixteen distinct 16-byte bank groups (rocprofv3
// SQ_LDS_BANK_CONFLICT reads 0 for this layout, 2.0e7 for an XOR with
// ((r >> 1) ^ (r >> 3)) & 3, 6.1e7 unswizzled, on the 3120x16384x4096 GEMM).
// ---------------------------------------------------------------------------
constexpr int kPBK = 64;  // bytes of K per stage

__device__ __forceinline__ int pswz(int r) { return (r >> 2) & 3; }

// s_waitcnt limiting only the vector-memory counter to n (n < 64); s_waitcnt
// limiting only the LDS counter to 0.
#define JO_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 15) | (((n) >> 4) << 14))
#define JO_WAIT_LDS0() __builtin_amdgcn_s_waitcnt(0xC07F)

template <int PER>
__device__ __forceinline__ void wait_loads(int later) {
  if (later >= 3)
    JO_WAIT_VM(3 * PER);
  else if (later == 2)
    JO_WAIT_VM(2 * PER);
  else if (later == 1)
    JO_WAIT_VM(PER);
  else
    JO_WAIT_VM(0);
}

// Direct loads of one stage: BM rows of A then BN rows of B^T, 64 bytes each,
// written by (BM + BN) / 16 wave instructions of 1 KB (16 rows, four lanes per
// row); slot L fills stage bytes L * 1024 .. +1024 and belongs to wave L % NW.
template <int BM, int BN, int NW>
struct PipeLoads {
  static constexpr int kSlots = (BM + BN) / 16;
  static constexpr int kPerWave = (kSlots + NW - 1) / NW;
  static constexpr bool kEven = kSlots % NW == 0;
  const uint8_t* base[kPerWave];  // wave-uniform: the tile's first row of A or B^T
  uint32_t off[kPerWave];         // this lane's 16-byte chunk of each slot at K offset 0
  bool last;                      // the wave owns a slot kPerWave - 1 (always when kEven)
};

// Epilogue of a wave's K loop, shared by the pipelined kernels. The LDS of
// the K loop's ring (at least 128 padded output rows) is free once every wave
// has passed the first barrier below.
template <class OutTag, int BM, int BN, int NW, int MI>
__device__ __forceinline__ void store_tile(const GemmArgs& g, uint8_t* smem,
                                           const f32x16 (&acc)[MI][BN / (NW / 2) / 32], int wm,
                                           int wn, int m0, int n0) {
  constexpr int WCOLS = BN / (NW / 2);
  constexpr int J = WCOLS / 32;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int fr = lane & 31, fh = lane >> 5;
  // Subtile (i, j) element e of a lane is row
  // m = m0 + wm*128 + i*32 + lane%32, column n = n0 + wn*WCOLS + j*32 +
  // (e/4)*8 + (lane/32)*4 + e%4. The finished values go through LDS (free
  // after the K loop) one 128-row half at a time, so that every row leaves
  // as whole lines of 16-byte lane stores: stored straight from the MFMA
  // layout (8 bytes per lane, 32 rows per wave store) the lines were written
  // back part-filled, measured 2.4-4.5x the output bytes in WRITE_SIZE.
  constexpr int kRowBytes = BN * 2 + 16;  // padded LDS row: 8-byte writes of 32 rows spread over the banks
  float sam[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) sam[i] = g.sa[min(m0 + wm * 128 + i * 32 + fr, g.M - 1)];
  float sbq[J][4][4], bq[J][4][4];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = min(n0 + wn * WCOLS + j * 32 + q * 8 + fh * 4, g.N - 4);  // N % 8 == 0
      const u32x4 sbv = ld16(g.sb + n);
      u32x4 b4{0u, 0u, 0u, 0u};
      if (g.bias) {
        const u32x2 braw = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(g.bias) + n);
        b4 = u32x4{braw.x, braw.y, 0u, 0u};
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        sbq[j][q][t] = elem<F32>(sbv, t);
        bq[j][q][t] = g.bias ? elem<OutTag>(b4, t) : 0.f;
      }
    }
  constexpr int kT = NW * 64;
  constexpr int kChunksPerRow = BN * 2 / 16;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    __syncthreads();  // the ring (or the previous half) is no longer read
    if (wm == half) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float o[8];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              o[t] = __builtin_fmaf(sam[i], acc[i][j][q * 4 + t] * sbq[j][q][t], bq[j][q][t]);
              o[t + 4] = 0.f;
            }
            const u32x4 pk = pack<OutTag>(o);
            const int rl = i * 32 + fr, cl = wn * WCOLS + j * 32 + q * 8 + fh * 4;
            *reinterpret_cast<u32x2*>(smem + rl * kRowBytes + cl * 2) = u32x2{pk.x, pk.y};
          }
    }
    __syncthreads();
    const int rows = half == 0 ? 128 : BM - 128;
    for (int c = tid; c < rows * kChunksPerRow; c += kT) {
      const int rl = c / kChunksPerRow, ch = c % kChunksPerRow;
      const int m = m0 + half * 128 + rl, n = n0 + ch * 8;
      if (m < g.M && n < g.N)
        st16_nt(static_cast<uint16_t*>(g.out) + static_cast<int64_t>(m) * g.ldo + n,
                *reinterpret_cast<const u32x4*>(smem + rl * kRowBytes + ch * 16));
    }
  }
}

// One output tile's K loop and epilogue for a wave holding MI row blocks of 32
// (rows wm*128 .. wm*128 + 32*MI - 1 of the tile) and WCOLS columns.
template <class OutTag, int BM, int BN, int NW, int NST, int MI>
__device__ __forceinline__ void fp8_gemm_pipe_tile(const GemmArgs& g, uint8_t* smem,
                                                   const PipeLoads<BM, BN, NW>& ld, int wave,
                                                   int wm, int wn, int m0, int n0) {
  using Loads = PipeLoads<BM, BN, NW>;
  constexpr int WCOLS = BN / (NW / 2);  // wave tile columns
  constexpr int J = WCOLS / 32;         // n-subtiles of 32 per wave
  constexpr int kStage = (BM + BN) * kPBK;
  static_assert(J >= 1 && MI >= 2 && MI <= 4, "tile shape");
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int stages = g.K / kPBK;
  auto issue = [&](int s) {
    uint8_t* base = smem + (s % NST) * kStage;
    const int kb = s * kPBK;
#pragma unroll
    for (int i = 0; i < Loads::kPerWave; ++i)
      if (Loads::kEven || i + 1 < Loads::kPerWave || ld.last)
        __builtin_amdgcn_global_load_lds(ld.base[i] + (ld.off[i] + kb), (__attribute__((address_space(3))) void*)(base + (wave + i * NW) * 1024), 16, 0, 0);
  };

  f32x16 acc[MI][J];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int fr = lane & 31, fh = lane >> 5;
  // LDS byte offsets of this lane's fragment chunks (same in every stage).
  int offa[MI][2], offb[J][2];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int r = wm * 128 + i * 32 + fr;
#pragma unroll
    for (int h = 0; h < 2; ++h) offa[i][h] = r * kPBK + (((fh * 2 + h) ^ pswz(r)) << 4);
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int r = wn * WCOLS + j * 32 + fr;
#pragma unroll
    for (int h = 0; h < 2; ++h) offb[j][h] = BM * kPBK + r * kPBK + (((fh * 2 + h) ^ pswz(r)) << 4);
  }

  auto read_frags = [&](int s, i32x8 (&af)[MI], i32x8 (&bf)[J]) {
    const uint8_t* st = smem + (s % NST) * kStage;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(st + offb[j][0]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(st + offb[j][1]);
      bf[j] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(st + offa[i][0]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(st + offa[i][1]);
      af[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
  };
  // Wait for this wave's loads of the stage being synced (with `later`
  // younger stages still allowed in flight) and its LDS reads, then meet the
  // other waves: that stage is complete in LDS, and every wave has finished
  // reading the stage before it. A bare s_barrier: a fenced barrier would
  // also wait for the loads of the later stages.
  auto sync_stage = [&](int later) {
    // On its own, outside the branch below: the compiler then knows that no
    // LDS read is pending after it and lets the MFMAs of the current
    // fragments run while the next stage's reads are in flight.
    __builtin_amdgcn_sched_barrier(0);  // the waits stay after the previous stage's MFMAs
    JO_WAIT_LDS0();
    if (Loads::kEven || ld.last)
      wait_loads<Loads::kPerWave>(later);
    else
      wait_loads<Loads::kPerWave - 1>(later);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // Software pipeline: at the start of stage s the wave waits for its LDS
  // reads (stage s's fragments) and for its own loads of stage s+1, then meets
  // the other waves: stage s+1 is complete in LDS, and every wave holds its
  // stage-s fragments, so the ring slot of stage s is free. It refills that
  // slot with stage s+NST, starts reading stage s+1's fragments into the
  // other register set and runs all of stage s's MFMAs while they arrive.
  for (int s = 0; s < NST && s < stages; ++s) issue(s);
  sync_stage(min(stages - 1, NST - 1));
  i32x8 af0[MI], bf0[J], af1[MI], bf1[J];
  read_frags(0, af0, bf0);
  // B first: the accumulator is the transposed tile, so a lane holds one
  // output row (m = lane % 32 of the subtile) and, per group of four
  // registers, four consecutive columns — stored as one 8-byte chunk.
  auto mfmas = [&](i32x8 (&af)[MI], i32x8 (&bf)[J]) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j) acc[i][j] = mfma32(bf[j], af[i], acc[i][j]);
  };
  // While stage s+NST exists, NST-2 younger stages stay in flight at the
  // sync: a constant wait.
  auto steady = [&](int s, i32x8 (&af)[MI], i32x8 (&bf)[J], i32x8 (&an)[MI], i32x8 (&bn)[J]) {
    // With 256-row tiles the first KB MFMAs of the stage go out before the
    // barrier (their fragments are this wave's own), so the matrix cores are
    // busy while the waves meet (4096^3: 67.4 -> 65.5 us on MI355X; with
    // 224-row tiles it measured 1-2% slower and is not done).
    constexpr int KB = BM == 256 ? 2 : 0;
    if constexpr (KB > 0) {
      __builtin_amdgcn_sched_barrier(0);
      JO_WAIT_LDS0();
      if (Loads::kEven || ld.last)
        wait_loads<Loads::kPerWave>(NST - 2);
      else
        wait_loads<Loads::kPerWave - 1>(NST - 2);
#pragma unroll
      for (int q = 0; q < KB; ++q) acc[q / J][q % J] = mfma32(bf[q % J], af[q / J], acc[q / J][q % J]);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    } else {
      sync_stage(NST - 2);
    }
    issue(s + NST);
    read_frags(s + 1, an, bn);
#pragma unroll
    for (int q = KB; q < MI * J; ++q) acc[q / J][q % J] = mfma32(bf[q % J], af[q / J], acc[q / J][q % J]);
    // Interleave: one MFMA, then two of the next stage's LDS reads (issuing
    // every read first measured 5-10% slower than this order).
#pragma unroll
    for (int q = KB; q < MI * J; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    }
  };
  auto drain = [&](int s, i32x8 (&af)[MI], i32x8 (&bf)[J], i32x8 (&an)[MI], i32x8 (&bn)[J]) {
    if (s + 1 < stages) {
      sync_stage(min(stages - 2 - s, NST - 2));
      if (s + NST < stages) issue(s + NST);
      read_frags(s + 1, an, bn);
    }
    mfmas(af, bf);
  };
  int s = 0;
  for (; s + 1 + NST < stages; s += 2) {
    steady(s, af0, bf0, af1, bf1);
    steady(s + 1, af1, bf1, af0, bf0);
  }
  for (; s < stages; s += 2) {
    drain(s, af0, bf0, af1, bf1);
    if (s + 1 < stages) drain(s + 1, af1, bf1, af0, bf0);
  }

  static_assert(128 * (BN * 2 + 16) <= NST * kStage, "epilogue staging fits the ring");
  store_tile<OutTag, BM, BN, NW, MI>(g, smem, acc, wm, wn, m0, n0);
}

template <class OutTag, int BM, int BN, int NW, int NST>
__device__ __forceinline__ void fp8_gemm_pipe_body(const GemmArgs& g) {
  using Loads = PipeLoads<BM, BN, NW>;
  static_assert(BM == 256 || BM == 224, "tile rows");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NST * (BM + BN) * kPBK];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  // BM = 256: a 2 x NW/2 grid of 128 x WCOLS wave tiles (even waves rows
  // 0-127, odd waves rows 128-255). BM = 224: waves 0 .. NW/2-1 take rows
  // 0-127 (four row blocks), the others rows 128-223 (three): a workgroup's
  // waves are spread round-robin over the CU's four SIMDs, so with NW = 8
  // each SIMD runs one wave of each kind, 7 row blocks where a 256-row tile
  // gives it 8.
  const int wm = BM == 256 ? (wave & 1) : wave / (NW / 2);
  const int wn = BM == 256 ? (wave >> 1) : wave % (NW / 2);
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  // Lane p of a slot fills row +p/4, chunk position p%4 with the global chunk
  // that belongs there. Rows beyond M (N) read row M-1 (N-1); they are never
  // stored. Addresses are a wave-uniform 64-bit tile base plus a 32-bit lane
  // offset (the host keeps 256 rows of A and B^T under 4 GB), which saves the
  // VGPRs of 64-bit per-lane pointers.
  Loads ld;
#pragma unroll
  for (int i = 0; i < Loads::kPerWave; ++i) {
    const int slot = wave + i * NW;
    const bool is_a = slot < BM / 16;
    const int r = (is_a ? slot : slot - BM / 16) * 16 + lane / 4;
    const int row = is_a ? min(m0 + r, g.M - 1) - m0 : min(n0 + r, g.N - 1) - n0;
    ld.base[i] = is_a ? g.a + static_cast<int64_t>(m0) * g.lda : g.b + static_cast<int64_t>(n0) * g.ldb;
    ld.off[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(is_a ? g.lda : g.ldb) +
                (((lane & 3) ^ pswz(r)) * 16);
  }
  ld.last = Loads::kEven || wave + (Loads::kPerWave - 1) * NW < Loads::kSlots;
  if constexpr (BM == 256) {
    fp8_gemm_pipe_tile<OutTag, BM, BN, NW, NST, 4>(g, smem, ld, wave, wm, wn, m0, n0);
  } else {
    if (wm == 0)
      fp8_gemm_pipe_tile<OutTag, BM, BN, NW, NST, 4>(g, smem, ld, wave, wm, wn, m0, n0);
    else
      fp8_gemm_pipe_tile<OutTag, BM, BN, NW, NST, 3>(g, smem, ld, wave, wm, wn, m0, n0);
  }
}

// The body lives in a device function: with the lambdas above directly in a
// kernel template over NW, the host compiler emits no launch stub for it.
template <class OutTag, int BM, int BN, int NW, int NST>
__global__ __launch_bounds__(NW * 64, 8 / NW) void fp8_gemm_pipe_kernel(const GemmArgs g) {
  fp8_gemm_pipe_body<OutTag, BM, BN, NW, NST>(g);
}

template <class OutTag, int BM, int BN, int NW, int NST>
void launch_pipe(const GemmArgs& g, hipStream_t stream) {
  hipLaunchKernelGGL((fp8_gemm_pipe_kernel<OutTag, BM, BN, NW, NST>),
                     dim3((g.N + BN - 1) / BN, (g.M + BM - 1) / BM), dim3(NW * 64), 0, stream, g);
}

// ---------------------------------------------------------------------------
// 128-byte-stage kernel (K % 128 == 0), the default for 8-wave tiles: the
// tile and wave layout of the pipelined kernel, but K advances in 128-byte
// stages through two LDS slots of (BM + BN) x 128 bytes. A wave's 1 KB direct
// load then covers eight whole 128-byte lines (eight lanes per row) where a
// 64-byte stage covers sixteen half lines. The loads are what bounds the K
// loop (a timing-only copy of the 64-byte kernel without them ran 4096^3 in
// 48 instead of 65 us), and the vector L1 stalls on its pending misses to L2:
// whole lines halve the L1 -> L2 requests for the same bytes (rocprofv3
// TCP_TCC_READ_REQ) and took 4096^3 from 67.7 to 61.2 us. Per stage s, one
// barrier:
//   MFMAs of the first 64-byte half    | reads of the second half's fragments
//   wait for those reads and for this wave's loads of stage s+1; barrier
//   MFMAs of the second half | loads of stage s+2 into the slot of stage s
//   (every wave holds its fragments now), reads of stage s+1's first half.
// LDS rows are 128 bytes; chunk c of row r sits at chunk position
// c ^ ((r >> 1) & 7): the sixteen consecutive rows a 16-lane group reads with
// one ds_read_b128 then fall in sixteen distinct 16-byte bank groups.
// ---------------------------------------------------------------------------
constexpr int kQBK = 128;  // bytes of K per stage

__device__ __forceinline__ int qswz(int r) { return (r >> 1) & 7; }

// Direct loads of one stage: BM rows of A then BN rows of B^T, 128 bytes
// each, written by (BM + BN) / 8 wave instructions of 1 KB (8 rows, eight
// lanes per row); slot L fills stage bytes L * 1024 .. +1024 and belongs to
// wave L % NW.
template <int BM, int BN, int NW>
struct PairLoads {
  static constexpr int kSlots = (BM + BN) / 8;
  static constexpr int kPerWave = (kSlots + NW - 1) / NW;
  static constexpr bool kEven = kSlots % NW == 0;
  const uint8_t* base[kPerWave];  // wave-uniform: the tile's first row of A or B^T
  uint32_t off[kPerWave];         // this lane's 16-byte chunk of each slot at K offset 0
  bool last;                      // the wave owns a slot kPerWave - 1 (always when kEven)
};

// NBS: B stages go through a ring of NBS slots beside A's two, so B loads run
// NBS - 1 stages ahead and A loads one (NBS = 3 for one-round grids, below).
template <class OutTag, int BM, int BN, int NW, int MI, int NBS>
__device__ __forceinline__ void fp8_gemm_pair_tile(const GemmArgs& g, uint8_t* smem,
                                                   const PairLoads<BM, BN, NW>& ld, int wave,
                                                   int wm, int wn, int m0, int n0) {
  using Loads = PairLoads<BM, BN, NW>;
  constexpr int WCOLS = BN / (NW / 2);  // wave tile columns
  constexpr int J = WCOLS / 32;         // n-subtiles of 32 per wave
  // Ring layout. NBS = 2: slot t % 2 holds stage t's A rows then its B rows.
  // NBS = 3: two A slots, then three B slots.
  constexpr int kASlot = NBS == 2 ? (BM + BN) * kQBK : BM * kQBK;
  constexpr int kBSlot = NBS == 2 ? (BM + BN) * kQBK : BN * kQBK;
  constexpr int kBBase = NBS == 2 ? BM * kQBK : 2 * BM * kQBK;
  constexpr int PER = Loads::kPerWave;
  constexpr int NB = BN / 8 / NW;  // B loads of a wave a stage: the last NB of its slots
  static_assert(J >= 1 && MI >= 2 && MI <= 4, "tile shape");
  static_assert((NBS == 2 || NBS == 3) && (BN / 8) % NW == 0, "B ring");
  static_assert(128 * (BN * 2 + 16) <= (2 * BM + NBS * BN) * kQBK, "epilogue staging fits the rings");
  const int lane = threadIdx.x % kWave;
  const int stages = g.K / kQBK;
  // Load i of this wave is A (slot index below BM / 8; a wave's A loads come
  // first in its slot order) or B; stage t of it goes to ring slot t % 2 or
  // t % NBS.
  auto is_a = [&](int i) { return wave + i * NW < BM / 8; };
  auto issue_one = [&](int t, int i) {
    if (Loads::kEven || i + 1 < PER || ld.last) {
      if constexpr (NBS == 2)
        __builtin_amdgcn_global_load_lds(ld.base[i] + (ld.off[i] + t * kQBK), (__attribute__((address_space(3))) void*)(smem + (t & 1) * kASlot + (wave + i * NW) * 1024), 16, 0, 0);
      else
        __builtin_amdgcn_global_load_lds(ld.base[i] + (ld.off[i] + t * kQBK), (__attribute__((address_space(3))) void*)(is_a(i) ? smem + (t & 1) * kASlot + (wave + i * NW) * 1024 : smem + kBBase + (t % NBS) * kBSlot + (wave + i * NW - BM / 8) * 1024), 16, 0, 0);
    }
  };
  // The loads issued in stage s's second half: A of stage s + 2 and B of
  // stage s + NBS.
  auto issue_batch_one = [&](int s, int i) {
    if constexpr (NBS == 2)
      issue_one(s + 2, i);
    else if (is_a(i))
      issue_one(s + 2, i);
    else if (s + NBS < stages)
      issue_one(s + NBS, i);
  };

  f32x16 acc[MI][J];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment rows are wm*128 + i*32 + lane%32 (A) and wn*WCOLS + j*32 +
  // lane%32 (B): all differ from lane%32 by multiples of 16, so they share
  // its swizzle, and row block i (j) sits i*32 (j*32) rows after block 0.
  const int fr = lane & 31, fh = lane >> 5;
  const int q = qswz(fr);
  int offa[2][2], offb[2][2];  // [half of the stage][chunk of the pair]
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int pos = ((k * 4 + fh * 2 + h) ^ q) << 4;
      offa[k][h] = (wm * 128 + fr) * kQBK + pos;
      offb[k][h] = kBBase + (wn * WCOLS + fr) * kQBK + pos;
    }
  auto read_frags = [&](int s, int k, i32x8 (&af)[MI], i32x8 (&bf)[J]) {
    const uint8_t* st = smem + (s & 1) * kASlot;
    const uint8_t* sb = NBS == 2 ? st : smem + (s % NBS) * kBSlot;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(sb + offb[k][0] + j * 32 * kQBK);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(sb + offb[k][1] + j * 32 * kQBK);
      bf[j] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(st + offa[k][0] + i * 32 * kQBK);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(st + offa[k][1] + i * 32 * kQBK);
      af[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
  };
  // Fragment f of half k of stage s: B block f (f < J), else A block f - J.
  auto read_one = [&](int s, int k, int f, i32x8 (&af)[MI], i32x8 (&bf)[J]) {
    const uint8_t* st = (NBS == 2 || f >= J) ? smem + (s & 1) * kASlot : smem + (s % NBS) * kBSlot;
    const int off = f < J ? offb[k][0] + f * 32 * kQBK : offa[k][0] + (f - J) * 32 * kQBK;
    const int off2 = f < J ? offb[k][1] + f * 32 * kQBK : offa[k][1] + (f - J) * 32 * kQBK;
    const u32x4 lo = *reinterpret_cast<const u32x4*>(st + off);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(st + off2);
    const i32x8 v{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    if (f < J)
      bf[f] = v;
    else
      af[f - J] = v;
  };
  // Stage s's wait: this wave's LDS reads, and its loads up to stage s + 1's.
  // A of s + 1 came with the latest loads; with NBS = 3 only their tail, B of
  // s + 2, may stay in flight.
  auto wait_next = [&](int s) {
    JO_WAIT_LDS0();
    if (NBS == 3 && s + 2 < stages)
      JO_WAIT_VM(NB);
    else
      JO_WAIT_VM(0);
  };
  auto bare_barrier = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // B first: the accumulator is the transposed tile (a lane holds one output
  // row and, per group of four registers, four consecutive columns).
  auto mfma_q = [&](int qi, i32x8 (&af)[MI], i32x8 (&bf)[J]) {
    acc[qi / J][qi % J] = mfma32(bf[qi % J], af[qi / J], acc[qi / J][qi % J]);
  };

  i32x8 a0[MI], b0[J], a1[MI], b1[J];  // fragments of the first / second half of a stage
  // With 256-row tiles the first KB MFMAs of the second half go out before
  // the barrier (their fragments are this wave's own), so the matrix cores
  // are busy while the waves meet.
  constexpr int KB = BM == 256 ? 2 : 0;
  // Stage s with stage s+1 present (NEXT) and stage s+2 present (MORE).
  auto stage = [&](int s, auto next, auto more) {
    constexpr bool kNext = decltype(next)::value, kMore = decltype(more)::value;
    // First half: MFMAs on a0/b0 while the second half's fragments arrive.
    read_frags(s, 1, a1, b1);
#pragma unroll
    for (int qi = 0; qi < MI * J; ++qi) mfma_q(qi, a0, b0);
#pragma unroll
    for (int qi = 0; qi < MI * J; ++qi) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_next(s);
#pragma unroll
    for (int qi = 0; qi < KB; ++qi) mfma_q(qi, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kNext) bare_barrier();
    // Second half, in a fixed order: each MFMA followed by up to two of stage
    // s+2's loads (the first four MFMAs carry them) and one of stage s+1's
    // first-half fragments. Issuing all of the stage's loads at once after the
    // barrier measured 2-4% slower on 4096^3 and the 3120-row qkv / MLP-up
    // shapes (level on the one-round MLP-down and attention-out shapes).
    constexpr int NQ = MI * J - KB;  // MFMAs after the barrier
    constexpr int NF = J + MI;       // fragments of the next first half
#pragma unroll
    for (int t = 0; t < NQ; ++t) {
      mfma_q(KB + t, a1, b1);
      if constexpr (kMore) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
          if (2 * t + u < PER) issue_batch_one(s, 2 * t + u);
      }
      if constexpr (kNext) {
        if (t < NF) read_one(s + 1, 0, t, a0, b0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kNext) {
#pragma unroll
      for (int f = NQ; f < NF; ++f) read_one(s + 1, 0, f, a0, b0);
    }
    if constexpr (kMore) {
#pragma unroll
      for (int i = 2 * NQ; i < PER; ++i) issue_batch_one(s, i);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  using T = std::true_type;
  using F = std::false_type;
  // Prologue: stage 0, then what the second halves of stages -2 and -1 would
  // have issued (stage 1; with NBS = 3, A of 1 and B of 1 and 2, B before A
  // within a stage); stage 0 starts once its own loads are in.
  auto issue_part = [&](int t, bool a) {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (is_a(i) == a) issue_one(t, i);
  };
  // In flight after stage 0's loads: NB B loads per later B stage and this
  // wave's A loads of stage 1 (PER - NB; one fewer for a wave without a last
  // slot, which is always a B slot since every wave has NB of those).
  const bool full = Loads::kEven || ld.last;
  if constexpr (NBS == 2) {
    auto issue = [&](int t) {
#pragma unroll
      for (int i = 0; i < PER; ++i) issue_one(t, i);
    };
    auto wait_own = [&](int later) {
      JO_WAIT_LDS0();
      if (Loads::kEven || ld.last)
        wait_loads<PER>(later);
      else
        wait_loads<PER - 1>(later);
    };
    issue(0);
    if (stages > 1) issue(1);
    wait_own(stages > 1 ? 1 : 0);
  } else {
    issue_part(0, false);
    issue_part(0, true);
    if (stages >= 3) {
      issue_part(1, false);
      issue_part(1, true);
      issue_part(2, false);
      JO_WAIT_LDS0();
      if (full)
        JO_WAIT_VM(2 * NB + PER - NB);
      else
        JO_WAIT_VM(2 * NB + PER - NB - 1);
    } else if (stages == 2) {
#pragma unroll
      for (int i = 0; i < PER; ++i) issue_one(1, i);
      JO_WAIT_LDS0();
      if (full)
        JO_WAIT_VM(PER);
      else
        JO_WAIT_VM(PER - 1);
    } else {
      JO_WAIT_LDS0();
      JO_WAIT_VM(0);
    }
  }
  bare_barrier();
  read_frags(0, 0, a0, b0);
  int s = 0;
  for (; s + 2 < stages; ++s) stage(s, T{}, T{});
  if (s + 1 < stages) stage(s++, T{}, F{});
  stage(s, F{}, F{});

  store_tile<OutTag, BM, BN, NW, MI>(g, smem, acc, wm, wn, m0, n0);
}

// Output tile of this workgroup. The dispatcher hands workgroup id (linear
// over the grid, x fastest) to XCD id % 8, and each XCD has its own L2, so
// consecutive ids are spread over the XCDs and the tiles an XCD runs
// together should share operand rows. XCD x gets a contiguous range of a
// grouped order (groups of four tile rows, column by column inside a group):
// the ~32 tiles it runs at once are four tile rows by eight columns, twelve
// operand panels where the row-major order gives it two columns by sixteen
// rows, eighteen (3120x12288x4096 141.0 -> 137.5 us, 3120x4096x16384
// 180.6 -> 176.3 us, 4096^3 59.0 -> 58.1 us).
__device__ __forceinline__ void xcd_grouped_tile(int bm, int bn, int& m0, int& n0) {
  constexpr int kGroup = 4;
  const int ntn = gridDim.x, ntm = gridDim.y, tiles = ntn * ntm;
  const int id = blockIdx.y * ntn + blockIdx.x;
  const int x = id & 7;
  const int t = x * (tiles >> 3) + min(x, tiles & 7) + (id >> 3);  // a bijection of [0, tiles)
  const int grp = t / (kGroup * ntn);
  const int r0 = grp * kGroup;
  const int rows = min(kGroup, ntm - r0);
  const int w = t - grp * kGroup * ntn;
  m0 = (r0 + w % rows) * bm;
  n0 = (w / rows) * bn;
}

template <class OutTag, int BM, int BN, int NW, int NBS>
__device__ __forceinline__ void fp8_gemm_pair_body(const GemmArgs& g) {
  using Loads = PairLoads<BM, BN, NW>;
  static_assert(BM == 256 || BM == 224, "tile rows");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[(2 * BM + NBS * BN) * kQBK];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  // Wave tiles as in fp8_gemm_pipe_body.
  const int wm = BM == 256 ? (wave & 1) : wave / (NW / 2);
  const int wn = BM == 256 ? (wave >> 1) : wave % (NW / 2);
  int m0, n0;
  xcd_grouped_tile(BM, BN, m0, n0);

  // Lane p of a slot fills row +p/8, chunk position p%8 with the global chunk
  // that belongs there. Rows beyond M (N) read row M-1 (N-1); they are never
  // stored. Wave-uniform 64-bit tile bases plus 32-bit lane offsets (the host
  // keeps 256 rows of A and B^T under 4 GB).
  Loads ld;
#pragma unroll
  for (int i = 0; i < Loads::kPerWave; ++i) {
    const int slot = wave + i * NW;
    const bool is_a = slot < BM / 8;
    const int r = (is_a ? slot : slot - BM / 8) * 8 + lane / 8;
    const int row = is_a ? min(m0 + r, g.M - 1) - m0 : min(n0 + r, g.N - 1) - n0;
    ld.base[i] = is_a ? g.a + static_cast<int64_t>(m0) * g.lda : g.b + static_cast<int64_t>(n0) * g.ldb;
    ld.off[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(is_a ? g.lda : g.ldb) +
                (((lane & 7) ^ qswz(r)) * 16);
  }
  ld.last = Loads::kEven || wave + (Loads::kPerWave - 1) * NW < Loads::kSlots;
  if constexpr (BM == 256) {
    fp8_gemm_pair_tile<OutTag, BM, BN, NW, 4, NBS>(g, smem, ld, wave, wm, wn, m0, n0);
  } else {
    if (wm == 0)
      fp8_gemm_pair_tile<OutTag, BM, BN, NW, 4, NBS>(g, smem, ld, wave, wm, wn, m0, n0);
    else
      fp8_gemm_pair_tile<OutTag, BM, BN, NW, 3, NBS>(g, smem, ld, wave, wm, wn, m0, n0);
  }
}

template <class OutTag, int BM, int BN, int NW, int NBS>
__global__ __launch_bounds__(NW * 64, 8 / NW) void fp8_gemm_pair_kernel(const GemmArgs g) {
  fp8_gemm_pair_body<OutTag, BM, BN, NW, NBS>(g);
}

template <class OutTag, int BM, int BN, int NW, int NBS = 2>
void launch_pair(const GemmArgs& g, hipStream_t stream) {
  hipLaunchKernelGGL((fp8_gemm_pair_kernel<OutTag, BM, BN, NW, NBS>),
                     dim3((g.N + BN - 1) / BN, (g.M + BM - 1) / BM), dim3(NW * 64), 0, stream, g);
}

// ---------------------------------------------------------------------------
// Small-tile kernel, for grids the 8-wave 224/256-row tiles would leave
// mostly idle (a few hundred rows: the text stream's Fp8Linear calls; 224x256
// tiles give [256, 4096] 32 tiles for 256 CUs). NW waves on a BM x BN tile
// (64x64, 64x128, 128x128 or 128x192 with four, 128x256 with eight) in a
// WGM x NW/WGM grid of wave tiles (WGM = 2); the 96-column tiles give each
// wave 32 x 96 (128x96: four waves down the rows, WGM = 4; 64x96: two waves,
// WGM = 2, two workgroups to a CU's LDS); K advances in 128-byte stages (whole lines, the LDS layout of the
// 128-byte-stage kernel) through a ring of NST slots that direct loads fill
// NST-1 stages ahead; one barrier a stage.
// Its K loop streams (BM + BN) x 128 bytes a stage for BM x BN x 128 MACs, so
// it only pays where it brings CUs into play that the large tiles leave idle.
// ---------------------------------------------------------------------------
template <int BM, int BN, int NW>
struct SmallLoads {
  static constexpr int kSlots = (BM + BN) / 8;  // 1 KB wave loads (8 rows) a stage
  static constexpr int kPerWave = kSlots / NW;
  static_assert(kSlots % NW == 0, "load slots spread evenly over the waves");
  const uint8_t* base[kPerWave];  // wave-uniform: the tile's first row of A or B^T
  uint32_t off[kPerWave];         // this lane's 16-byte chunk of each slot at K offset 0
};

template <class OutTag, int BM, int BN, int NW, int NST, bool SPLIT, int WGM>
__device__ __forceinline__ void fp8_gemm_small_body(const GemmArgs& g) {
  constexpr int WROWS = BM / WGM, WCOLS = BN / (NW / WGM);  // wave tile
  constexpr int MI = WROWS / 32, J = WCOLS / 32;
  constexpr int kStage = (BM + BN) * kQBK;
  constexpr int kRowBytes = BN * 2 + 16;  // padded LDS row of the staged output tile
  constexpr int kChunksPerRow = BN * 2 / 16;
  using Loads = SmallLoads<BM, BN, NW>;
  constexpr int PER = Loads::kPerWave;
  static_assert(NW % WGM == 0 && WROWS % 32 == 0 && WCOLS % 32 == 0 && MI >= 1 && J >= 1 &&
                    BM * kRowBytes <= NST * kStage && NST >= 2 && NST <= 5,
                "tile shape");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NST * kStage];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave % WGM, wn = wave / WGM;
  int m0, n0;
  xcd_grouped_tile(BM, BN, m0, n0);

  // Lane p of load slot L fills row 8L + p/8 of the stage (A rows, then B^T
  // rows), chunk position p%8, with the global chunk that belongs there; rows
  // beyond M (N) read row M-1 (N-1) and are never stored.
  Loads ld;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int slot = wave + i * NW;
    const bool is_a = slot < BM / 8;
    const int r = (is_a ? slot : slot - BM / 8) * 8 + lane / 8;
    const int row = is_a ? min(m0 + r, g.M - 1) - m0 : min(n0 + r, g.N - 1) - n0;
    ld.base[i] = is_a ? g.a + static_cast<int64_t>(m0) * g.lda : g.b + static_cast<int64_t>(n0) * g.ldb;
    ld.off[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(is_a ? g.lda : g.ldb) +
                (((lane & 7) ^ qswz(r)) * 16);
  }
  // SPLIT: workgroup z of the grid's gridDim.z takes the z-th equal share of
  // the K stages and writes its partial product for the reduction kernel.
  const int stages = SPLIT ? g.K / kQBK / static_cast<int>(gridDim.z) : g.K / kQBK;
  const int s0 = SPLIT ? static_cast<int>(blockIdx.z) * stages : 0;
  auto issue = [&](int s) {
    uint8_t* dst = smem + (s % NST) * kStage;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      __builtin_amdgcn_global_load_lds(ld.base[i] + (ld.off[i] + (s0 + s) * kQBK),
                                       (__attribute__((address_space(3))) void*)(dst + (wave + i * NW) * 1024),
                                       16, 0, 0);
  };

  // Fragment rows wm*WROWS + i*32 + lane%32 (A) and wn*WCOLS + j*32 +
  // lane%32 (B): multiples of 32 apart, so they share lane%32's swizzle.
  const int fr = lane & 31, fh = lane >> 5;
  const int q = qswz(fr);
  int offa[2][2], offb[2][2];  // [half of the stage][chunk of the pair]
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int pos = ((k * 4 + fh * 2 + h) ^ q) << 4;
      offa[k][h] = (wm * WROWS + fr) * kQBK + pos;
      offb[k][h] = BM * kQBK + (wn * WCOLS + fr) * kQBK + pos;
    }
  f32x16 acc[MI][J];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  auto compute = [&](int s) {
    const uint8_t* st = smem + (s % NST) * kStage;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      i32x8 af[MI], bf[J];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(st + offb[k][0] + j * 32 * kQBK);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(st + offb[k][1] + j * 32 * kQBK);
        bf[j] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(st + offa[k][0] + i * 32 * kQBK);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(st + offa[k][1] + i * 32 * kQBK);
        af[i] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
      // B first: the accumulator is the transposed tile (as in store_tile).
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j) acc[i][j] = mfma32(bf[j], af[i], acc[i][j]);
    }
  };

  // At stage s the wave waits for its LDS reads (of stage s-1) and its own
  // loads of stage s (the younger stages stay in flight), then meets the other
  // waves: stage s is complete in LDS and every wave is done with the slot of
  // stage s-1, which then takes stage s+NST-1.
  for (int s = 0; s < NST - 1 && s < stages; ++s) issue(s);
  for (int s = 0; s < stages; ++s) {
    JO_WAIT_LDS0();
    wait_loads<PER>(min(stages - 1 - s, NST - 2));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (s + NST - 1 < stages) issue(s + NST - 1);
    compute(s);
  }

  if constexpr (SPLIT) {
    // The partial tile as fp32: a lane's four consecutive columns per group
    // are one 16-byte store, and a row's 32 columns of a block (128 bytes)
    // leave in the four stores of one (i, j) back to back. Plain stores: the
    // reduction reads them back right away.
    float* wz = g.ws + static_cast<int64_t>(blockIdx.z) * g.M * g.N;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int m = m0 + wm * WROWS + i * 32 + fr;
          const int n = n0 + wn * WCOLS + j * 32 + qq * 8 + fh * 4;
          // Each element through a scalar first: a bit_cast of a vector
          // element expression reads element 0 with this compiler.
          const float v0 = acc[i][j][qq * 4 + 0], v1 = acc[i][j][qq * 4 + 1];
          const float v2 = acc[i][j][qq * 4 + 2], v3 = acc[i][j][qq * 4 + 3];
          if (m < g.M && n < g.N)
            st16(wz + static_cast<int64_t>(m) * g.N + n,
                 u32x4{__builtin_bit_cast(uint32_t, v0), __builtin_bit_cast(uint32_t, v1),
                       __builtin_bit_cast(uint32_t, v2), __builtin_bit_cast(uint32_t, v3)});
        }
    return;
  }
  // Epilogue: the finished tile goes through LDS (free once every wave is past
  // the barrier) so that rows leave as whole 16-byte lane stores.
  float sam[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) sam[i] = g.sa[min(m0 + wm * WROWS + i * 32 + fr, g.M - 1)];
  float sbq[J][4][4], bq[J][4][4];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int n = min(n0 + wn * WCOLS + j * 32 + qq * 8 + fh * 4, g.N - 4);  // N % 8 == 0
      const u32x4 sbv = ld16(g.sb + n);
      u32x4 b4{0u, 0u, 0u, 0u};
      if (g.bias) {
        const u32x2 braw = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(g.bias) + n);
        b4 = u32x4{braw.x, braw.y, 0u, 0u};
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        sbq[j][qq][t] = elem<F32>(sbv, t);
        bq[j][qq][t] = g.bias ? elem<OutTag>(b4, t) : 0.f;
      }
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        float o[8];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          o[t] = __builtin_fmaf(sam[i], acc[i][j][qq * 4 + t] * sbq[j][qq][t], bq[j][qq][t]);
          o[t + 4] = 0.f;
        }
        const u32x4 pk = pack<OutTag>(o);
        const int rl = wm * WROWS + i * 32 + fr, cl = wn * WCOLS + j * 32 + qq * 8 + fh * 4;
        *reinterpret_cast<u32x2*>(smem + rl * kRowBytes + cl * 2) = u32x2{pk.x, pk.y};
      }
  __syncthreads();
  for (int c = tid; c < BM * kChunksPerRow; c += NW * kWave) {
    const int rl = c / kChunksPerRow, ch = c % kChunksPerRow;
    const int m = m0 + rl, n = n0 + ch * 8;
    if (m < g.M && n < g.N)
      st16_nt(static_cast<uint16_t*>(g.out) + static_cast<int64_t>(m) * g.ldo + n,
              *reinterpret_cast<const u32x4*>(smem + rl * kRowBytes + ch * 16));
  }
}

template <class OutTag, int BM, int BN, int NW, int NST, bool SPLIT, int WGM>
__global__ __launch_bounds__(NW * 64) void fp8_gemm_small_kernel(const GemmArgs g) {
  fp8_gemm_small_body<OutTag, BM, BN, NW, NST, SPLIT, WGM>(g);
}

// Split K, second pass: out[m, n] = epilogue of the sum over z of the
// partials ws[z, m, n], added in z order (so every run gives the same bits),
// eight columns a thread.
template <class OutTag>
__global__ __launch_bounds__(kBlock) void fp8_gemm_splitk_reduce(const GemmArgs g, int splits) {
  const int64_t cpr = g.N / 8;  // N % 8 == 0
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (c >= static_cast<int64_t>(g.M) * cpr) return;
  const int64_t m = c / cpr;
  const int n = static_cast<int>(c - m * cpr) * 8;
  const int64_t plane = static_cast<int64_t>(g.M) * g.N;
  const float* p = g.ws + m * g.N + n;
  float acc[8];
  {
    const u32x4 lo = ld16(p), hi = ld16(p + 4);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      acc[t] = elem<F32>(lo, t);
      acc[t + 4] = elem<F32>(hi, t);
    }
  }
  for (int z = 1; z < splits; ++z) {
    const u32x4 lo = ld16(p + z * plane), hi = ld16(p + z * plane + 4);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      acc[t] += elem<F32>(lo, t);
      acc[t + 4] += elem<F32>(hi, t);
    }
  }
  const float sa = g.sa[m];
  const u32x4 s0 = ld16(g.sb + n), s1 = ld16(g.sb + n + 4);
  u32x4 braw{0u, 0u, 0u, 0u};
  if (g.bias) braw = ld16(static_cast<const uint16_t*>(g.bias) + n);
  float o[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float sb = t < 4 ? elem<F32>(s0, t) : elem<F32>(s1, t - 4);
    o[t] = __builtin_fmaf(sa, acc[t] * sb, g.bias ? elem<OutTag>(braw, t) : 0.f);
  }
  st16_nt(static_cast<uint16_t*>(g.out) + m * g.ldo + n, pack<OutTag>(o));
}

template <class OutTag, int BM, int BN, int NW, int NST, int WGM = 2>
void launch_small(const GemmArgs& g, hipStream_t stream, int splits = 1) {
  const dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM, splits);
  if (splits == 1) {
    hipLaunchKernelGGL((fp8_gemm_small_kernel<OutTag, BM, BN, NW, NST, false, WGM>), grid,
                       dim3(NW * 64), 0, stream, g);
    return;
  }
  hipLaunchKernelGGL((fp8_gemm_small_kernel<OutTag, BM, BN, NW, NST, true, WGM>), grid, dim3(NW * 64),
                     0, stream, g);
  const int64_t chunks = static_cast<int64_t>(g.M) * (g.N / 8);
  hipLaunchKernelGGL((fp8_gemm_splitk_reduce<OutTag>), dim3(static_cast<unsigned>((chunks + kBlock - 1) / kBlock)),
                     dim3(kBlock), 0, stream, g, splits);
}

// CUs of the current device (queried once per device; 256, MI355X's count,
// if the query fails).
int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// One workgroup per CU at most (a single round of tiles). There the 224-row
// pair kernel runs its B loads two stages ahead (NBS = 3): with no second
// round to overlap, the lines wait longer (~530 cycles against ~360 on the
// multi-round shapes), and the extra stage of B lookahead measured
// 3120x4096x16384 178 -> 168 us and 3120x4096x4096 50.6 -> 48.1 us (three
// alternating runs, results bit-identical); on the multi-round shapes and
// the 256-row tiles (4096^3) it was 3-4% slower.
bool one_round(const GemmArgs& g, int bm, int bn) {
  const int64_t tiles = static_cast<int64_t>((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn);
  return tiles <= cu_count();
}

// Tile rows for the 8-wave x 256-column kernel: one workgroup per CU, so the
// time is about (rounds of workgroups over the CUs) x (row blocks per SIMD),
// 8 for a 256-row tile and 7 for a 224-row one. At M = 3120 (13 tiles of 256,
// 14 of 224) every deployment shape needs the same number of rounds with
// either height, and 224-row tiles measured 3120x12288x4096 185 -> 180 us,
// 3120x16384x4096 233 -> 224 us, 3120x4096x16384 198 -> 193 us.
int pick_tile_rows(int M, int N) {
  const int64_t cus = cu_count(), cols = (N + 255) / 256;
  auto cost = [&](int64_t bm) { return ((M + bm - 1) / bm * cols + cus - 1) / cus * (bm / 32); };
  return cost(224) < cost(256) ? 224 : 256;
}

// The default launch shape. The K loops are bound by the operand bytes each
// CU streams from L2 (~45 KB/us per CU for every kernel here), so the cost of
// a shape is (tiles per CU, rounded up) x (BM + BN) bytes per K byte: the 8-wave
// 224x256 or 256x256 tiles (pick_tile_rows) unless the small-tile kernel at
// 128x256, 128x192, 128x128, 128x96, 64x128, 64x96 or 64x64 streams fewer bytes on the
// busiest CU, as where the large tiles leave most CUs idle (ties go to the
// smaller tile: two 64x64 workgroups share a CU). The 96-column tiles cut
// N = 12288 into 128 columns of tiles, so 128 or 256 rows fill the 256 CUs.
// Measured on MI355X, M = 256: [256, 4096] x 4096 34.2 -> 11.4 us (64x64),
// [256, 12288] x 4096 42.4 -> 24.3 us (128x128) -> 22.0 us (128x96); M = 128,
// [128, 12288] x 4096 20.4 us (64x128) -> 17.9 us (64x96); M = 1024,
// [1024, 4096] x 16384 155.4 -> 86.4 us (128x128).
int auto_shape(int M, int N) {
  const int64_t cus = cu_count();
  auto cost = [&](int64_t bm, int64_t bn) {
    return ((M + bm - 1) / bm * ((N + bn - 1) / bn) + cus - 1) / cus * (bm + bn);
  };
  const int bm = pick_tile_rows(M, N);
  int shape = bm == 224 ? 3 : 0;
  int64_t best = cost(bm, 256);
  // Larger tiles first: a tie goes to the smaller one.
  const int small[7][3] = {{7, 128, 256}, {9, 128, 192}, {5, 128, 128}, {10, 128, 96},
                            {8, 64, 128}, {11, 64, 96}, {6, 64, 64}};
  for (const auto& t : small)
    if (cost(t[1], t[2]) <= best) {
      best = cost(t[1], t[2]);
      shape = t[0];
    }
  return shape;
}

// Split K, for few tiles and a long K (the text stream's MLP down: [256,
// 16384] x [16384, 4096] is 64 tiles of 128x128): S workgroups share each
// tile's K stages and write fp32 partials that a second kernel adds up in a
// fixed order (the same bits on every run) under the epilogue. Taken by the
// small-tile kernel at 128x128 or 64x64 when the caller passes a workspace of
// S x M x N x 4 bytes and it cuts the cost above by 15% or more: the busiest
// CU's operand bytes, plus the partials written and read back (they stay in
// the caches: counted at half an operand byte) and a fixed ~9 us for the
// second launch and the first one's tail (405 KB at the operand rate), fitted
// on MI355X: [64, 4096] x 16384 38.8 -> 22.5 us, [256, 4096] x 16384 39.2 ->
// 34.4 us, [512, 4096] x 16384 65.9 -> 51.7 us; [512, 4096] x 4096 stays
// unsplit (16.5 us; split in two, 20.6).
constexpr int64_t kSplitCap = int64_t{1} << 30;  // largest partial buffer a split uses

struct GemmPlan {
  int shape;
  int splits;
};

void shape_dims(int shape, int M, int N, int& bm, int& bn) {
  switch (shape) {
    case 5: bm = 128; bn = 128; break;
    case 6: bm = 64; bn = 64; break;
    case 7: bm = 128; bn = 256; break;
    case 8: bm = 64; bn = 128; break;
    case 9: bm = 128; bn = 192; break;
    case 10: bm = 128; bn = 96; break;
    case 11: bm = 64; bn = 96; break;
    default: bm = shape == 3 ? 224 : 256; bn = 256; break;
  }
  (void)M;
  (void)N;
}

int64_t split_bytes(int M, int N, int splits) {
  return splits > 1 ? static_cast<int64_t>(splits) * M * N * 4 : 0;
}

int64_t plan_cost(int M, int N, int K, int bm, int bn, int splits) {
  const int64_t cus = cu_count();
  const int64_t tiles = static_cast<int64_t>((M + bm - 1) / bm) * ((N + bn - 1) / bn);
  int64_t c = (tiles * splits + cus - 1) / cus * (bm + bn) * (K / splits);
  if (splits > 1) c += split_bytes(M, N, splits) / cus + 405 * 1024;
  return c;
}

GemmPlan plan_gemm(const GemmArgs& g, int64_t ws_bytes) {
  const int forced = launch_knob(JO_KNOB_GEMM_SHAPE);
  const int fsplit = launch_knob(JO_KNOB_GEMM_SPLIT);
  GemmPlan p{forced >= 0 ? forced : auto_shape(g.M, g.N), 1};
  const int64_t room = ws_bytes < kSplitCap ? ws_bytes : kSplitCap;
  auto split_ok = [&](int sp) {
    return g.K > 0 && g.K % (kQBK * sp) == 0 && split_bytes(g.M, g.N, sp) <= room;
  };
  if (fsplit >= 1) {
    if ((p.shape == 5 || p.shape == 6) && split_ok(fsplit)) p.splits = fsplit;
    return p;
  }
  if (forced >= 0) return p;
  int bm, bn;
  shape_dims(p.shape, g.M, g.N, bm, bn);
  const int64_t unsplit = plan_cost(g.M, g.N, g.K, bm, bn, 1);
  int64_t best = -1;
  GemmPlan split{p.shape, 1};
  const int cand[2][3] = {{5, 128, 128}, {6, 64, 64}};
  for (const auto& c : cand)
    for (int sp = 2; sp <= 8; sp *= 2)
      if (split_ok(sp)) {
        const int64_t cost = plan_cost(g.M, g.N, g.K, c[1], c[2], sp);
        if (best < 0 || cost < best) {
          best = cost;
          split = GemmPlan{c[0], sp};
        }
      }
  return (best >= 0 && best * 20 < unsplit * 17) ? split : p;
}

template <class OutTag>
int launch_gemm(const GemmArgs& g, hipStream_t stream, int64_t ws_bytes) {
  const dim3 grid((g.N + kBN - 1) / kBN, (g.M + kBM - 1) / kBM);
  // K == 0 takes the register-staged kernel, which loads no operand bytes
  // when K is 0 and stores the epilogue of a zero accumulator (the bias).
  const bool pipe_ok = g.K > 0 && g.K % kPBK == 0 && aligned(g.sb, 16) && (g.bias == nullptr || aligned(g.bias, 8)) &&
                       256 * (g.lda > g.ldb ? g.lda : g.ldb) + g.K <= int64_t{UINT32_MAX};
  // 8-wave 256-column tiles measured faster than two 4-wave 128-column
  // workgroups per CU at every deployment shape (3120x12288x4096: 199 -> 185
  // us, 3120x16384x4096: 257 -> 233 us). The JO_KNOB_GEMM_SHAPE override
  // 0|1|2|3|4|5|6|7|8|9|10|11 forces 256x256, 256x128, the register-staged
  // kernel, 224x256, 224x128, or the small-tile kernel at 128x128, 64x64,
  // 128x256, 64x128, 128x192, 128x96 or 64x96
  // (results are the same up to the fp32 accumulation order inside the
  // matrix cores).
  const GemmPlan plan = plan_gemm(g, ws_bytes);
  const int shape = plan.shape;
  const bool pair_ok = pipe_ok && g.K % kQBK == 0;
  if (pipe_ok && shape == 1)
    launch_pipe<OutTag, 256, 128, 4, 3>(g, stream);
  else if (pair_ok && shape == 0)
    launch_pair<OutTag, 256, 256, 8>(g, stream);
  else if (pair_ok && shape == 3 && one_round(g, 224, 256))
    launch_pair<OutTag, 224, 256, 8, 3>(g, stream);
  else if (pair_ok && shape == 3)
    launch_pair<OutTag, 224, 256, 8>(g, stream);
  else if (pipe_ok && shape == 0)
    launch_pipe<OutTag, 256, 256, 8, 4>(g, stream);
  else if (pipe_ok && shape == 3)
    launch_pipe<OutTag, 224, 256, 8, 4>(g, stream);
  else if (pipe_ok && shape == 4)
    launch_pipe<OutTag, 224, 128, 4, 3>(g, stream);
  else if (pair_ok && shape == 5)
    launch_small<OutTag, 128, 128, 4, 4>(g, stream, plan.splits);
  else if (pair_ok && shape == 6)
    launch_small<OutTag, 64, 64, 4, 4>(g, stream, plan.splits);
  else if (pair_ok && shape == 7)
    launch_small<OutTag, 128, 256, 8, 3>(g, stream);
  else if (pair_ok && shape == 8)
    launch_small<OutTag, 64, 128, 4, 4>(g, stream);
  else if (pair_ok && shape == 9)
    launch_small<OutTag, 128, 192, 4, 3>(g, stream);
  else if (pair_ok && shape == 10)
    launch_small<OutTag, 128, 96, 4, 4, 4>(g, stream);
  else if (pair_ok && shape == 11)
    launch_small<OutTag, 64, 96, 2, 4, 2>(g, stream);
  else
    hipLaunchKernelGGL((fp8_gemm_kernel<OutTag>), grid, dim3(kBlock), 0, stream, g);
  return launch_status("fp8_scaled_mm");
}

}  // namespace
}  // namespace jo

using namespace jo;

namespace {
int fp8_scaled_mm_impl(const void* mat_a, int64_t lda, const void* mat_b, int64_t ldb,
                       const float* scales_a, const float* scales_b, const void* bias, void* out,
                       int64_t ldo, int64_t M, int64_t N, int64_t K, int out_dtype,
                       void* workspace, int64_t workspace_bytes, void* stream) {
  const char* op = "fp8_scaled_mm";
  JO_REQUIRE(out_dtype == JO_DTYPE_BF16 || out_dtype == JO_DTYPE_F16,
             "out_dtype must be Half or BFloat16");
  JO_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX,
             "%s: bad shape", op);
  JO_REQUIRE(K % 16 == 0, "mat_a must be multiple of 16 bytes for memory alignment");
  JO_REQUIRE(N % 8 == 0, "out must be multiple of 16 bytes for memory alignment");
  JO_REQUIRE(lda >= K && ldb >= K && ldo >= N && lda % 16 == 0 && ldb % 16 == 0 && ldo % 8 == 0,
             "%s: row strides must cover the rows and keep 16-byte alignment", op);
  if (M == 0 || N == 0) return JO_OK;
  // With K == 0 no operand byte is read (torch hands zero-size views over as
  // null pointers), and the output is the epilogue of a zero accumulator.
  JO_REQUIRE((K == 0 || (mat_a && mat_b)) && scales_a && scales_b && out, "%s: null pointer", op);
  JO_REQUIRE(aligned(mat_a, 16) && aligned(mat_b, 16) && aligned(out, 16),
             "%s: operands must be 16-byte aligned", op);
  JO_REQUIRE(workspace_bytes >= 0 && (workspace_bytes == 0 || (workspace && aligned(workspace, 16))),
             "%s: workspace must be 16-byte aligned (or 0 bytes)", op);
  GemmArgs g{static_cast<const uint8_t*>(mat_a), static_cast<const uint8_t*>(mat_b), scales_a,
             scales_b, bias, out, lda, ldb, ldo, static_cast<int>(M), static_cast<int>(N),
             static_cast<int>(K), static_cast<float*>(workspace)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  return out_dtype == JO_DTYPE_BF16 ? launch_gemm<BF16>(g, st, workspace_bytes)
                                    : launch_gemm<F16>(g, st, workspace_bytes);
}
}  // namespace

extern "C" int jo_fp8_scaled_mm(const void* mat_a, int64_t lda, const void* mat_b, int64_t ldb,
                                const float* scales_a, const float* scales_b, const void* bias,
                                void* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                int out_dtype, void* stream) {
  return fp8_scaled_mm_impl(mat_a, lda, mat_b, ldb, scales_a, scales_b, bias, out, ldo, M, N, K,
                            out_dtype, nullptr, 0, stream);
}

extern "C" int jo_fp8_scaled_mm_ws(const void* mat_a, int64_t lda, const void* mat_b,
                                   int64_t ldb, const float* scales_a, const float* scales_b,
                                   const void* bias, void* out, int64_t ldo, int64_t M, int64_t N,
                                   int64_t K, int out_dtype, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  return fp8_scaled_mm_impl(mat_a, lda, mat_b, ldb, scales_a, scales_b, bias, out, ldo, M, N, K,
                            out_dtype, workspace, workspace_bytes, stream);
}

// Allocation-free variant: the split-K partials go to this file-scope device
// array instead of a caller's workspace. Each GPU the library runs on holds
// its own copy (kScratchBytes) until the process ends. Host code never uses
// the array's name as an address (it is a host-side stand-in there): the
// device address comes from hipGetSymbolAddress, once per device.
constexpr int64_t kScratchBytes = int64_t{32} << 20;
static __device__ __align__(256) float scratch[kScratchBytes / 4];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];

// The current device's address of `scratch`, looked up on the first call on
// that device (with it current) and kept.
int scratch_address(void** out) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("fp8_scaled_mm_noalloc: no usable current device (%s)", hipGetErrorString(ge));
    return JO_ERR_HIP;
  }
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("fp8_scaled_mm_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                dev, hipGetErrorString(e));
      return JO_ERR_HIP;
    }
    g_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return JO_OK;
}
}  // namespace

extern "C" int64_t jo_fp8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return 0;
  GemmArgs g{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, K, K, N,
             static_cast<int>(M), static_cast<int>(N), static_cast<int>(K)};
  const GemmPlan p = plan_gemm(g, kSplitCap);
  return split_bytes(g.M, g.N, p.splits);
}

extern "C" int jo_fp8_scaled_mm_noalloc(const void* mat_a, int64_t lda, const void* mat_b,
                                        int64_t ldb, const float* scales_a,
                                        const float* scales_b, const void* bias, void* out,
                                        int64_t ldo, int64_t M, int64_t N, int64_t K,
                                        int out_dtype, void* stream) {
  const int64_t need = jo_fp8_scaled_mm_workspace_bytes(M, N, K);
  JO_REQUIRE(need <= kScratchBytes,
             "fp8_scaled_mm_noalloc: the split-K partials of [%lld, %lld] x %lld need %lld bytes, "
             "more than the %lld-byte static scratch (jo_fp8_scaled_mm_ws takes a workspace of "
             "any size)",
             static_cast<long long>(M), static_cast<long long>(K), static_cast<long long>(N),
             static_cast<long long>(need), static_cast<long long>(kScratchBytes));
  void* ws = nullptr;
  if (need > 0) {
    const int st = scratch_address(&ws);
    if (st != JO_OK) return st;
  }
  return fp8_scaled_mm_impl(mat_a, lda, mat_b, ldb, scales_a, scales_b, bias, out, ldo, M, N, K,
                            out_dtype, ws, need, stream);
}
