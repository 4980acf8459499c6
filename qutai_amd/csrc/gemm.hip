// GEMM entry points of libqutai_amd (C ABI).  The argument meaning, the
// dtype rules and the validation follow the reference GEMM boundary
// `cuda.gemm` (src/qutai/backends/cuda.py:305-362) and its kernel signature
// (src/qutai/backends/cuda/gemm.cu:35, `(a, b, out, M, K, N, sa, sb, ta, tb,
// accumulate)`); kernel choice is MI355X-specific.
#include <cstdlib>
#include <string>

#include "gemm_kernel.h"
#include "gemm_pingpong.h"
#include "gemm_short.h"

#include <algorithm>
#include "qutai_amd.h"

using namespace qa;

namespace {

template <class Kern>
__global__ void __launch_bounds__(Kern::NT) gemm_entry(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) char smem[Kern::LDS_BYTES];
  Kern::run(p, smem);
}

template <class Kern>
__global__ void __launch_bounds__(Kern::NT) pingpong_entry(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) char smem[Kern::LDS_BYTES];
  Kern::run(p, smem);
}

template <class Kern>
__global__ void __launch_bounds__(Kern::NT, Kern::MIN_BLOCKS) short_entry(ShortArgs p) {
  __shared__ __attribute__((aligned(16))) char smem[Kern::LDS_BYTES];
  Kern::run(p, smem);
}

// fp64 GEMM: plain 32x32 SIMT tiles, 2x2 outputs per thread (not an MFMA
// target; kept for the float64 storage contract of the boundary).
__global__ void __launch_bounds__(256) gemm_f64(const double* a, const double* b, double* out, int64_t M,
                                                int64_t K, int64_t N, int64_t sa, int64_t sb, int ta, int tb,
                                                int accumulate, int64_t tiles_n, int64_t tiles_m) {
  __shared__ double As[32][33], Bs[32][33];
  int x = threadIdx.x & 15, y = threadIdx.x >> 4;
  int64_t id = blockIdx.x;
  int64_t z = id / (tiles_m * tiles_n), t = id % (tiles_m * tiles_n);
  int64_t tm = t / tiles_n, tn = t % tiles_n;
  a += z * sa;
  b += z * sb;
  out += z * M * N;
  double c[2][2] = {{0, 0}, {0, 0}};
  for (int64_t k0 = 0; k0 < K; k0 += 32) {
    for (int dy = 0; dy < 2; dy++)
      for (int dx = 0; dx < 2; dx++) {
        int64_t r = tm * 32 + y + dy * 16, k = k0 + x + dx * 16;
        As[y + dy * 16][x + dx * 16] = (r < M && k < K) ? a[ta ? k * M + r : r * K + k] : 0.0;
        int64_t kk = k0 + y + dy * 16, cc = tn * 32 + x + dx * 16;
        Bs[y + dy * 16][x + dx * 16] = (kk < K && cc < N) ? b[tb ? cc * K + kk : kk * N + cc] : 0.0;
      }
    __syncthreads();
    for (int k = 0; k < 32; k++) {
      double a0 = As[y][k], a1 = As[y + 16][k], b0 = Bs[k][x], b1 = Bs[k][x + 16];
      c[0][0] = __dadd_rn(c[0][0], __dmul_rn(a0, b0));
      c[0][1] = __dadd_rn(c[0][1], __dmul_rn(a0, b1));
      c[1][0] = __dadd_rn(c[1][0], __dmul_rn(a1, b0));
      c[1][1] = __dadd_rn(c[1][1], __dmul_rn(a1, b1));
    }
    __syncthreads();
  }
  for (int dy = 0; dy < 2; dy++)
    for (int dx = 0; dx < 2; dx++) {
      int64_t r = tm * 32 + y + dy * 16, cc = tn * 32 + x + dx * 16;
      if (r < M && cc < N) {
        double v = c[dy][dx];
        if (accumulate) v += out[r * N + cc];
        out[r * N + cc] = v;
      }
    }
}

// Operand re-layout into the workspace: dst[z][o][i] = src[z*stride + o*inner + i]
// for i < inner (converted to the compute type; fp32 -> bf16 rounds to
// nearest even) and 0 in the padding up to `pitch`.  Used when an fp32
// operand feeds the bf16 MFMA path (mixed inputs, autocast) or when the
// operand's rows are not 16-byte aligned.  Each thread fills PREP_CHUNKS
// 16-byte chunks of the destination (E = 8 bf16 or 4 fp32 values; pitch is
// a multiple of E) with loads that are contiguous across a wavefront, all in
// flight before the 16-byte stores (one per thread measured fastest: the
// grid then keeps every CU's wave slots busy).  One launch covers the rows [row_base, row_base + rows) with
// 32-bit chunk indices (rows * pitch / E < 2^31; the host splits larger
// operands into several launches), the row's (batch, row) pair in 64 bits.
struct PrepareArgs {
  const void* src;
  void* dst;
  int64_t row_base, outer, stride;
  uint32_t rows, inner, pitch;
};

// One destination chunk i (16 bytes) of the re-layout, loaded and packed.
template <bool SRC_BF16, bool DST_BF16>
__device__ __forceinline__ u32x4 prepare_load(const PrepareArgs& a, uint32_t i) {
  constexpr int E = DST_BF16 ? 8 : 4;
  const uint32_t per_row = a.pitch / E;
  const uint32_t r = i / per_row, c0 = (i - r * per_row) * E;
  const int64_t row = a.row_base + r, z = row / a.outer, o = row - z * a.outer;
  const int64_t at = z * a.stride + o * a.inner + c0;
  if constexpr (SRC_BF16 && DST_BF16) {
    if (c0 + E <= a.inner) {
      // a whole chunk inside the row: one 16-byte load at the element's own
      // (2-byte) alignment -- unaligned global loads are enabled on this
      // platform, and the compiler emits the same for an unaligned memcpy
      u32x4 w;
      __builtin_memcpy(&w, (const char*)a.src + at * 2, 16);
      return w;
    }
  }
  float v[E];
#pragma unroll
  for (int t = 0; t < E; t++) {
    v[t] = 0.f;
    if (c0 + t < a.inner)
      v[t] = SRC_BF16 ? bf16_to_f32(((const bf16_t*)a.src)[at + t]) : ((const float*)a.src)[at + t];
  }
  if constexpr (DST_BF16)
    return u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
  else
    return u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
}

// PREP_CHUNKS chunks per thread, 256 apart (a wavefront's loads stay
// contiguous).
constexpr int PREP_CHUNKS = 1;
template <bool SRC_BF16, bool DST_BF16>
__device__ __forceinline__ void prepare_chunks(const PrepareArgs& a, uint32_t block) {
  constexpr int E = DST_BF16 ? 8 : 4;
  const uint32_t total = a.rows * (a.pitch / E);
  u32x4 w[PREP_CHUNKS];
#pragma unroll
  for (int q = 0; q < PREP_CHUNKS; q++) {
    const uint32_t i = (block * PREP_CHUNKS + q) * 256u + threadIdx.x;
    if (i < total) w[q] = prepare_load<SRC_BF16, DST_BF16>(a, i);
  }
#pragma unroll
  for (int q = 0; q < PREP_CHUNKS; q++) {
    const uint32_t i = (block * PREP_CHUNKS + q) * 256u + threadIdx.x;
    if (i < total) global_store((char*)a.dst + (a.row_base * (a.pitch / E) + i) * 16, w[q]);
  }
}

template <bool SRC_BF16, bool DST_BF16>
__global__ void __launch_bounds__(256) prepare_operand(PrepareArgs a) {
  prepare_chunks<SRC_BF16, DST_BF16>(a, blockIdx.x);
}

// Split-K reduction: out[b][e] = sum over s of part[b * splits + s][e] in
// order s = 0, 1, ... (fp32), plus the old output when accumulating, one
// rounding to the output type.  The partials hold rows of `cols` elements;
// out's rows are `ldc` apart (a column window of a wider output).
__global__ void splitk_reduce(const float* part, void* out, int64_t n, int64_t total, int splits, int accumulate,
                              int out_bf16, int64_t cols, int64_t ldc) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / n, e = i - b * n;
    const float* src = part + b * splits * n + e;
    float acc = 0.f;
    for (int s = 0; s < splits; s++) acc += src[s * n];
    const int64_t row = e / cols, at = (b * (n / cols) + row) * ldc + (e - row * cols);
    if (accumulate) acc += out_bf16 ? bf16_to_f32(((const bf16_t*)out)[at]) : ((const float*)out)[at];
    if (out_bf16) ((bf16_t*)out)[at] = f32_to_bf16(acc);
    else ((float*)out)[at] = acc;
  }
}

// Column remainder of at most 8 columns with a K-major A (the last r
// columns of a 256 q + r wide product): a workgroup of RWAVES waves computes
// RWAVES * RROWS output rows.  It stages B's r columns for KC values of k at
// a time in LDS as fp32 (zero beyond K; each element rounded to the compute
// type first, so an fp32 B read in place gives what its re-laid-out bf16
// copy would), while every wave's 16-byte loads of its rows of A for the
// same KC values are in flight:
// lane l sums the 16-byte chunks l, l + 64, ... of its row in K order
// (KC is a multiple of 64 chunks, so the staging does not change that
// order), then a fixed xor tree over the lanes, then the GEMM epilogue's
// accumulate and rounding.  A is a planned operand: rows 16-byte aligned and
// zero-padded to its pitch, so no 16-byte chunk crosses the allocation.  B is
// read at its source dtype and pitch (b_bf16, kb: K-major), r columns from
// column `col`.
constexpr int RWAVES = 4, RROWS = 4, RBLOCK = RWAVES * RROWS, RKC = 1024;
struct RemainderArgs {
  const void* a;
  const void* b;
  void* out;
  int64_t M, K, lda, ldb, ldc, col;
  int r, out_bf16, accumulate;
};

template <bool BF16, bool B_BF16, bool KB>
__device__ __forceinline__ void remainder_block(const RemainderArgs& p, int64_t block, float* cols) {
  constexpr int E = BF16 ? 8 : 4;
  constexpr int NC = RKC / E / 64;  // 16-byte chunks per lane and row in one staged block
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = block * RBLOCK + wave * RROWS;
  const int r = p.r;
  float acc[RROWS][8];
#pragma unroll
  for (int i = 0; i < RROWS; i++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[i][j] = 0.f;
  for (int64_t kc = 0; kc < p.K; kc += RKC) {
    // this block's A chunks first (in flight while B's columns are staged)
    const int64_t chunks = (std::min<int64_t>(p.K - kc, RKC) + E - 1) / E;
    u32x4 w[RROWS][NC];
#pragma unroll
    for (int i = 0; i < RROWS; i++)
#pragma unroll
      for (int q = 0; q < NC; q++) {
        const int64_t m = row0 + i, c = lane + 64 * q;
        w[i][q] = u32x4{0u, 0u, 0u, 0u};
        if (m < p.M && c < chunks) w[i][q] = *(const u32x4*)((const char*)p.a + (m * p.lda + kc + c * E) * (BF16 ? 2 : 4));
      }
    __syncthreads();  // the previous block's columns are no longer read
    // cols[j][k - kc] = B(k, col + j) in the compute type; MN-major B: the
    // r columns of one k are neighbours, so a wave reads whole row segments
    // (four loads in flight per thread: the elements of an MN-major B sit
    // in as many rows, one cache line each)
    for (int t0 = 0; t0 < r * RKC; t0 += 4 * 64 * RWAVES) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int t = t0 + u * 64 * RWAVES + tid;
        const int j = KB ? t / RKC : t % r, kk = KB ? t % RKC : t / r;
        const int64_t k = kc + kk;
        v[u] = 0.f;
        if (t < r * RKC && k < p.K) {
          const int64_t at = KB ? (p.col + j) * p.ldb + k : k * p.ldb + p.col + j;
          v[u] = B_BF16 ? bf16_to_f32(((const bf16_t*)p.b)[at]) : ((const float*)p.b)[at];
          if (BF16 && !B_BF16) v[u] = bf16_to_f32(f32_to_bf16(v[u]));
        }
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int t = t0 + u * 64 * RWAVES + tid;
        const int j = KB ? t / RKC : t % r, kk = KB ? t % RKC : t / r;
        if (t < r * RKC) cols[j * RKC + kk] = v[u];
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NC; q++) {
      const int64_t c = lane + 64 * q;
      if (c >= chunks) break;
      // one column's values at a time (few registers, so the re-layout
      // workgroups that share this kernel keep their occupancy); every
      // (row, column) sum still runs over its chunk's elements in order
#pragma unroll
      for (int j = 0; j < 8; j++) {
        if (j >= r) break;
        float bv[E];
#pragma unroll
        for (int e = 0; e < E; e += 4) {
          const f32x4 v = *(const f32x4*)(cols + j * RKC + c * E + e);
          bv[e] = v[0];
          bv[e + 1] = v[1];
          bv[e + 2] = v[2];
          bv[e + 3] = v[3];
        }
#pragma unroll
        for (int i = 0; i < RROWS; i++) {
#pragma unroll
          for (int e = 0; e < E; e++) {
            const uint32_t h = w[i][q][BF16 ? e >> 1 : e];
            const float x = BF16 ? __uint_as_float((e & 1) ? (h & 0xffff0000u) : (h << 16)) : __uint_as_float(h);
            acc[i][j] = __builtin_fmaf(x, bv[e], acc[i][j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RROWS; i++) {
    const int64_t m = row0 + i;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (j >= r) break;
      float v = acc[i][j];
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
      if (lane == j && m < p.M) {
        const int64_t at = m * p.ldc + j;
        if (p.accumulate) v += p.out_bf16 ? bf16_to_f32(((const bf16_t*)p.out)[at]) : ((const float*)p.out)[at];
        if (p.out_bf16) ((bf16_t*)p.out)[at] = f32_to_bf16(v);
        else ((float*)p.out)[at] = v;
      }
    }
  }
}

template <bool BF16, bool B_BF16, bool KB>
__global__ void __launch_bounds__(64 * RWAVES, 3) remainder_columns(RemainderArgs p) {
  __shared__ __attribute__((aligned(16))) float cols[8 * RKC];
  remainder_block<BF16, B_BF16, KB>(p, blockIdx.x, cols);
}

// B's re-layout and the column remainder in one launch: they are
// independent (the remainder reads B at its source pitch), so the first
// `rem_blocks` workgroups compute remainder rows while the others copy B;
// the large-tile launch that reads the re-laid-out B follows on the stream.
template <bool SRC_BF16, bool BF16, bool KB>
__global__ void __launch_bounds__(256, 3) prepare_remainder(PrepareArgs a, RemainderArgs p, unsigned rem_blocks) {
  __shared__ __attribute__((aligned(16))) float cols[8 * RKC];
  if (blockIdx.x < rem_blocks) remainder_block<BF16, SRC_BF16, KB>(p, blockIdx.x, cols);
  else prepare_chunks<SRC_BF16, BF16>(a, blockIdx.x - rem_blocks);
}

// Kernel configurations: (BM x BN, WM x WN waves, BK, LDS stages, staging).
//   L8D2: 256x256, 8 waves (2 per SIMD), BK 64 (bf16) / 32 (fp32), two-stage
//         direct-to-LDS ring, the next stage's copies spread over the k-steps
//   L8R : 256x256, 8 waves, same K step, register staging
//   L4D2: 256x256, 4 waves (one per SIMD, 128x128 per wave), two-stage ring
//   S   : 128x128, 4 waves, BK 32 / 16, four-stage ring (small grids, short K)
//   S2  : 128x128, 4 waves, BK 32 / 16, two-stage ring (bf16, K <= 64: four per CU)
//   N   : 256x64, 4 waves (N <= 64), BK 64 / 32, two-stage ring, A's copies
//         streamed (nontemporal: one column tile reads every A row once)
//         when A's rows start on 128-byte lines and A exceeds 256 MiB
//   W   : 64x256, 4 waves (M <= 64), BK 32 / 16, four-stage ring
//   H   : 256x128, 8 waves 4x2 (64x64 per wave), BK 64, three-stage ring
//         (grids of 256x256 tiles that would leave half the CUs idle)
//   T, U: 192x256 (8 waves 2x4, 96x64 per wave) and 256x192 (4x2, 64x96),
//         BK 64, two-stage ring, bf16 only (a grid of 256x256 tiles just
//         short of the CU count, e.g. 5632 x 2048: 176 tiles -> 240)
//   R   : short-K row strips (gemm_short.h): bf16 NT with K <= 64, a 128-row
//         block of A held in registers, 128-column chunks of B through a
//         two-slot LDS ring, 128-byte row segments staged through LDS
enum Tile { TILE_L8D2, TILE_L8R, TILE_L4D2, TILE_S, TILE_N, TILE_W, TILE_H, TILE_T, TILE_U, TILE_S2, TILE_R, TILE_P,
            TILE_COUNT };

template <bool F32, bool TA, bool TB, int BM, int BN, int WM, int WN, int BK, int ST, bool DMA, bool SWIGLU = false,
          bool GATHER_B = false, bool STREAM_A = false>
hipError_t launch_cfg(GemmArgs p, hipStream_t stream) {
  typedef GemmKernel<F32, TA, TB, BM, BN, WM, WN, BK, ST, DMA, SWIGLU, GATHER_B, STREAM_A> Kern;
  int64_t tiles_n = (p.N + Kern::BNO - 1) / Kern::BNO;
  if (p.groups == 0) p.tiles_m = (int)((p.M + BM - 1) / BM);
  int64_t blocks = (int64_t)p.tiles_m * tiles_n * (p.groups ? 1 : p.batch);
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gemm_entry<Kern>, dim3((unsigned)blocks), dim3(Kern::NT), 0, stream, p);
  return hipGetLastError();
}

int forced_tile();

// Tile P: the ping-pong kernel (gemm_pingpong.h) for plain bf16 products
// with K a multiple of 64; other calls take L8D2, whose results it matches
// bit for bit.  Unforced, a 256x256 choice in the NN, NT and TT forms runs
// it (1-3% faster on 4096^3 and 8192-class shapes; TN is equal or 1% slower
// and keeps GemmKernel).
bool pingpong_fits(const GemmArgs& p) {
  return p.K > 0 && p.K % 64 == 0 && p.groups == 0 && p.k_split <= 1 && p.k_head == 0 && !p.group_k;
}
template <bool TA, bool TB>
hipError_t launch_pingpong(GemmArgs p, hipStream_t stream) {
  typedef PingPong<TA, TB> Kern;
  p.tiles_m = (int)((p.M + 255) / 256);
  const int64_t blocks = (int64_t)p.tiles_m * ((p.N + 255) / 256) * p.batch;
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pingpong_entry<Kern>, dim3((unsigned)blocks), dim3(Kern::NT), 0, stream, p);
  return hipGetLastError();
}

// Streamed A copies for the thin tile: A's rows (K-major) or k-rows
// (MN-major), in every batch entry and second K segment, start on 128-byte
// lines, and A spans at least the 256 MiB of the memory-side cache (an
// operand that fits there is cheaper to read with plain loads, which find
// the lines a previous kernel or call left there: a 16384 x 1408 A of a
// 32-column product ran 19.5 us plain against 21.6 us streamed).
bool stream_a(const GemmArgs& p, int64_t es) {
  auto line = [](int64_t bytes) { return bytes % 128 == 0; };
  const int64_t span = p.a_bytes > 0 ? p.a_bytes
                       : (p.batch > 1 && p.sa > 0 ? p.batch * p.sa : (p.groups ? 0 : p.M * p.lda)) * es;
  return span >= (int64_t(256) << 20) && (uintptr_t)p.a % 128 == 0 && line(p.lda * es) && line(p.sa * es) &&
         (p.k_head == 0 || (uintptr_t)p.a_tail % 128 == 0);
}

template <bool F32, bool TA, bool TB>
hipError_t launch_tile(Tile tile, GemmArgs p, hipStream_t stream) {
  constexpr int KB = F32 ? 16 : 32;  // K per stage of the four-stage rings
  constexpr int KR = F32 ? 32 : 64;  // K per stage of the two-stage rings
  switch (tile) {
    case TILE_P:
      if constexpr (!F32)
        if (pingpong_fits(p)) return launch_pingpong<TA, TB>(p, stream);
      return launch_cfg<F32, TA, TB, 256, 256, 2, 4, KR, 2, true>(p, stream);
    case TILE_L8R: return launch_cfg<F32, TA, TB, 256, 256, 2, 4, KR, 2, false>(p, stream);
    case TILE_L4D2: return launch_cfg<F32, TA, TB, 256, 256, 2, 2, KR, 2, true>(p, stream);
    case TILE_S: return launch_cfg<F32, TA, TB, 128, 128, 2, 2, KB, 4, true>(p, stream);
    case TILE_S2: return launch_cfg<F32, TA, TB, 128, 128, 2, 2, KB, 2, true>(p, stream);
    case TILE_N:
      // one column tile: every A row is read by one workgroup, streamed
      // (nontemporal copies, K per stage 64 bf16 / 32 fp32 = 128 bytes of a
      // K-major row) where A's rows start on 128-byte lines, so that every
      // copy reads whole lines, and A is larger than the memory-side cache;
      // otherwise the same tile with plain copies
      if (stream_a(p, F32 ? 4 : 2))
        return launch_cfg<F32, TA, TB, 256, 64, 4, 1, KR, 2, true, false, false, true>(p, stream);
      return launch_cfg<F32, TA, TB, 256, 64, 4, 1, KR, 2, true>(p, stream);
    case TILE_W: return launch_cfg<F32, TA, TB, 64, 256, 1, 4, KB, 4, true>(p, stream);
    case TILE_H: return launch_cfg<F32, TA, TB, 256, 128, 4, 2, KR, 3, true>(p, stream);
    case TILE_T:
      if constexpr (F32) return launch_cfg<F32, TA, TB, 256, 256, 2, 4, KR, 2, true>(p, stream);
      else return launch_cfg<F32, TA, TB, 192, 256, 2, 4, KR, 2, true>(p, stream);
    case TILE_U:
      if constexpr (F32) return launch_cfg<F32, TA, TB, 256, 256, 2, 4, KR, 2, true>(p, stream);
      else return launch_cfg<F32, TA, TB, 256, 192, 4, 2, KR, 2, true>(p, stream);
    default:
      // the ping-pong kernel where it measured faster (bit-identical results)
      if constexpr (!F32 && !(TA && !TB))
        if (forced_tile() < 0 && pingpong_fits(p)) return launch_pingpong<TA, TB>(p, stream);
      return launch_cfg<F32, TA, TB, 256, 256, 2, 4, KR, 2, true>(p, stream);
  }
}

// Grouped-K products whose B K rows are read through GemmArgs::b_rows: the
// two-stage direct-to-LDS tiles (192x256 and 256x192 for bf16, else 256x256).
template <bool F32>
hipError_t launch_gathered_k(Tile tile, const GemmArgs& p, hipStream_t stream) {
  constexpr int KR = F32 ? 32 : 64;
  if constexpr (!F32) {
    if (tile == TILE_T) return launch_cfg<F32, true, false, 192, 256, 2, 4, KR, 2, true, false, true>(p, stream);
    if (tile == TILE_U) return launch_cfg<F32, true, false, 256, 192, 4, 2, KR, 2, true, false, true>(p, stream);
  }
  return launch_cfg<F32, true, false, 256, 256, 2, 4, KR, 2, true, false, true>(p, stream);
}

template <bool F32>
hipError_t launch_mma(Tile tile, bool ta, bool tb, const GemmArgs& p, hipStream_t stream) {
  if (ta) return tb ? launch_tile<F32, true, true>(tile, p, stream) : launch_tile<F32, true, false>(tile, p, stream);
  return tb ? launch_tile<F32, false, true>(tile, p, stream) : launch_tile<F32, false, false>(tile, p, stream);
}

// compute units of the current device (cached per device)
int64_t cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Tile choice for an M x N output (batch of them) over K; thin outputs use
// the 256x64 / 64x256 shapes.  QUTAI_AMD_GEMM_TILE=<L8D2|L8R|L4D2|S|N|W|H|T|U|S2|R>
// overrides the choice (tuning and tests; R applies only where the short-K
// strip kernel does, other calls then take L8D2).
int forced_tile() {
  static int forced = [] {
    const char* v = getenv("QUTAI_AMD_GEMM_TILE");
    if (!v) return -1;
    const char* names[TILE_COUNT] = {"L8D2", "L8R", "L4D2", "S", "N", "W", "H", "T", "U", "S2", "R", "P"};
    for (int i = 0; i < TILE_COUNT; i++)
      if (std::string(v) == names[i]) return i;
    return -1;
  }();
  return forced;
}

Tile pick_tile(int64_t M, int64_t N, int64_t batch, bool bf16, double* cost);

Tile choose_tile(int64_t M, int64_t N, int64_t K, int64_t batch, bool bf16) {
  if (forced_tile() >= 0) return (Tile)forced_tile();
  if (N <= 64) return TILE_N;
  if (M <= 64) return TILE_W;
  // K <= 64 (bf16; the attention score product S = Q K^T with K = the head
  // size) is bound by writing the output: a two-stage ring halves the LDS
  // of the four-stage one, so four workgroups fit per CU instead of two
  // (config 3's S product 336 -> 291 us)
  if (bf16 && K <= 64) return TILE_S2;
  if (K <= 128) return TILE_S;
  // Wave-quantisation cost of the large tiles, in units of one full round of
  // 256x256 tiles over the CUs (per unit of K).  Measured on this GPU (bf16,
  // 4096^3 and the decoder / ragged shapes): a full round of 256x128 tiles
  // (one per CU) costs 0.665, a full round of 128x128 tiles (two per CU)
  // 0.70, and a partial round of at most one 128x128 tile per CU 0.5; a
  // round of 192x256 / 256x192 tiles (bf16) 0.9; a partial round of the
  // others costs as much as a full one.  Ties (within 3%) go to 256x128,
  // then 256x192, 192x256, 256x256.
  return pick_tile(M, N, batch, bf16, nullptr);
}

// The large-tile choice of choose_tile and its cost (rounds of 256x256 tiles
// over the CUs, per unit of K).
Tile pick_tile(int64_t M, int64_t N, int64_t batch, bool bf16, double* cost) {
  const int64_t cus = cu_count();
  auto rounds = [cus](int64_t tiles) { return (double)(tiles / cus + (tiles % cus ? 1 : 0)); };
  const int64_t mt = (M + 255) / 256, nt = (N + 255) / 256, ms = (M + 127) / 128, ns = (N + 127) / 128;
  const int64_t nl = mt * nt * batch, nh = mt * ns * batch, nsm = ms * ns * batch;
  const double cost_l = rounds(nl);
  const double cost_h = 0.665 * rounds(nh);
  const int64_t rs = nsm % (2 * cus);
  const double cost_s = 0.70 * (double)(nsm / (2 * cus)) + (rs == 0 ? 0.0 : rs <= cus ? 0.5 : 0.70);
  const double cost_t = bf16 ? 0.9 * rounds((M + 191) / 192 * nt * batch) : 1e30;
  const double cost_u = bf16 ? 0.9 * rounds(mt * ((N + 191) / 192) * batch) : 1e30;
  const double best = std::min({cost_l, cost_h, cost_s, cost_t, cost_u});
  Tile pick = TILE_S;
  double chosen = cost_s;
  if (cost_h <= best * 1.03) pick = TILE_H, chosen = cost_h;
  else if (cost_u <= best * 1.03) pick = TILE_U, chosen = cost_u;
  else if (cost_t <= best * 1.03) pick = TILE_T, chosen = cost_t;
  else if (cost_l <= best * 1.03) pick = TILE_L8D2, chosen = cost_l;
  if (cost) *cost = chosen;
  return pick;
}

// Column remainder: an output N = 256 q + r wide with 0 < r <= 64, whose last
// r columns cost the large tiles about a round of their own (4095 x 4097:
// 272 tiles of 256x256 or 352 of 256x192 for 256 CUs), runs as two launches:
// the first 256 q columns on the large tiles and the last r on the thin
// 256x64 tile, which splits K when its tiles fill few CUs (priced at 0.3 of a
// round).  Returns the first launch's width, or 0 for one launch.  Each
// output element still sums K through the same MFMA chain (split K sums its
// chunks in order), so results stay bit-repeatable.
int64_t column_split(int64_t M, int64_t N, int64_t K, int64_t batch, bool bf16) {
  if (forced_tile() >= 0 || batch != 1 || M <= 64 || K <= 128 || N < 512) return 0;
  const int64_t r = N % 256;
  if (r == 0 || r > 64) return 0;
  double full = 0.0, main = 0.0;
  pick_tile(M, N, 1, bf16, &full);
  pick_tile(M, N - r, 1, bf16, &main);
  return main + 0.3 < full * 0.97 ? N - r : 0;
}

// Split-K for plain products whose tiles fill at most a quarter of the CU
// slots over a long K (e.g. 1024 x 2048 outputs with K = 32768; a two-way
// split of half-empty grids measured slower): the K
// range is cut into chunks of a multiple of 64 elements, each chunk's fp32
// partial product goes to the workspace and one pass sums them.
// QUTAI_AMD_SPLITK=<n> forces n chunks (tuning and tests; read per call).
size_t split_bytes(int64_t rows, int64_t cols, int64_t batch, int splits) {
  return ((size_t)splits * batch * rows * cols * 4 + 255) / 256 * 256;
}

// rows of an output tile (the M extent a grouped launch counts tiles in)
int tile_rows(Tile tile) {
  switch (tile) {
    case TILE_S:
    case TILE_S2: return 128;
    case TILE_T: return 192;
    case TILE_W: return 64;
    default: return 256;
  }
}

// Tile of a grouped (per-expert rows) launch: 256x64 for thin outputs, else
// 256x256 or, for bf16, 256x192 when that takes fewer weighted rounds over
// the CUs (a round of 256x192 tiles costs 0.9 of a 256x256 one, as in
// choose_tile).  The M tile count is estimated as ceil(rows / 256) plus half
// a partial tile per group.  The 256x128 / 128x128 tiles measured slower on
// config 5's experts and are not considered.  Config 5's down product
// (cols 2048): 256x192 109 us against 123 us for 256x256.
Tile grouped_tile(int64_t rows, int64_t cols, int groups, bool bf16) {
  if (forced_tile() >= 0) return (Tile)forced_tile();
  if (cols <= 64) return TILE_N;
  if (!bf16) return TILE_L8D2;
  const int64_t cus = cu_count();
  auto rounds = [cus](int64_t tiles) { return (double)(tiles / cus + (tiles % cus ? 1 : 0)); };
  const int64_t tiles_m = (rows + 255) / 256 + groups / 2;
  const double cost_l = rounds(tiles_m * ((cols + 255) / 256));
  const double cost_u = 0.9 * rounds(tiles_m * ((cols + 191) / 192));
  return cost_u < cost_l * 0.97 ? TILE_U : TILE_L8D2;
}

int64_t tile_count(Tile tile, int64_t rows, int64_t cols, int64_t batch) {
  int64_t bm = 256, bn = 256;
  if (tile == TILE_S) bm = bn = 128;
  else if (tile == TILE_H) bn = 128;
  else if (tile == TILE_T) bm = 192;
  else if (tile == TILE_U) bn = 192;
  else if (tile == TILE_N) bn = 64;
  else if (tile == TILE_W) bm = 64;
  return ((rows + bm - 1) / bm) * ((cols + bn - 1) / bn) * batch;
}

// A plain product whose tiles fill at most a quarter of the tile slots over
// K >= 4096 splits K.  For bf16 the tile and the split count are then chosen
// together: each candidate (256x256, 256x128, 128x128) takes the most chunks
// that fit its slots, at most 8 and at least 1024 of K each, and is priced as
// its rounds of tiles over the chunk (the wave-quantisation costs of
// choose_tile, a full 256x256 round being 113 us per 4096 of K on this GPU)
// plus the partial sums' HBM traffic (s writes, s reads and one output write
// of rows x cols fp32 at 5 TB/s).  Measured: the decoder head's dX (1024 x
// 2048 outputs, K = 32768) takes 256x256 in 8 chunks, 158 -> 137 us; the
// K/V projections' weight gradients (512 x 2048, K = 4096) take 128x128 in
// 4 chunks, 28 -> 24 us.  The tile may change; a forced tile does not.
int choose_split(int64_t rows, int64_t cols, int64_t inner, int64_t batch, Tile* tile, bool bf16, int64_t* chunk) {
  const int64_t cus = cu_count();
  const int64_t tiles = tile_count(*tile, rows, cols, batch);
  const int64_t slots = (*tile == TILE_S ? 2 : 1) * cus;
  int64_t s = 1;
  const char* forced = getenv("QUTAI_AMD_SPLITK");
  if (forced && atoi(forced) > 0) {
    s = atoi(forced);
  } else if (batch == 1 && tiles * 4 <= slots && inner >= 4096) {
    s = std::min<int64_t>(8, slots / tiles);
    if (bf16 && forced_tile() < 0) {
      double best = 1e30;
      for (Tile t : {TILE_L8D2, TILE_H, TILE_S}) {
        const int64_t n = tile_count(t, rows, cols, 1), per = (t == TILE_S ? 2 : 1) * cus;
        const int64_t st = std::max<int64_t>(1, std::min<int64_t>({8, per / n, inner / 1024}));
        const int64_t units = n * st, r = (units + cus - 1) / cus;
        double rounds;
        if (t == TILE_L8D2) rounds = (double)r;
        else if (t == TILE_H) rounds = 0.665 * (double)r;
        else {
          const int64_t rs = units % (2 * cus);
          rounds = 0.70 * (double)(units / (2 * cus)) + (rs == 0 ? 0.0 : rs <= cus ? 0.5 : 0.70);
        }
        const double k_chunk = (double)((inner + st - 1) / st);
        const double reduce_us = st > 1 ? (2.0 * st + 1) * rows * cols * 4 / 5.0e6 : 0.0;
        const double cost = rounds * k_chunk * (113.0 / 4096) + reduce_us;
        if (cost < best) {
          best = cost;
          *tile = t;
          s = st;
        }
      }
    }
  } else if (batch == 1 && (*tile == TILE_N || *tile == TILE_W) && tiles * 4 <= cus && inner >= 512) {
    // a thin output (<= 64 columns or rows) over a few 256-wide blocks, e.g.
    // a router's logits or a column remainder: latency-bound tiles, so K
    // chunks down to 64 (up to 16 of them) put the idle CUs to work
    // (8192 x 2048 x 8 logits of an 8-expert router: 32 workgroups -> 256;
    // the last column of 4095 x 1000 x 4097: 16 -> 256)
    s = std::min<int64_t>({16, cus / tiles, (inner + 63) / 64});
  }
  if (s <= 1 || inner < 128) return 1;
  const int64_t c = ((inner + s - 1) / s + 63) / 64 * 64;
  s = (inner + c - 1) / c;
  if (s <= 1) return 1;
  *chunk = c;
  return (int)s;
}

// How one operand reaches the kernel: in place, or re-laid out in the
// workspace (dtype change and/or zero-padded 16-byte-aligned rows).
struct Operand {
  const void* ptr;
  int64_t ld, stride, src_stride;
  bool copy;
  int64_t outer, inner, pitch, batches;
  size_t bytes;  // workspace bytes when copied
};

Operand plan_operand(const void* p, int dtype, bool compute_bf16, int64_t outer, int64_t inner, int64_t batch,
                     int64_t stride) {
  const int64_t E = compute_bf16 ? 8 : 4;
  const int64_t es = compute_bf16 ? 2 : 4;
  bool same = (dtype == QA_BF16) == compute_bf16;
  bool aligned = ((uintptr_t)p % 16 == 0) && (inner % E == 0) && (batch <= 1 || stride % E == 0);
  Operand o = {p, inner, stride, stride, !(same && aligned), outer, inner, inner, 1, 0};
  if (o.copy) {
    o.pitch = (inner + E - 1) / E * E;
    o.batches = (stride == 0 || batch <= 1) ? 1 : batch;
    o.ld = o.pitch;
    o.stride = stride == 0 ? 0 : outer * o.pitch;
    o.bytes = (size_t)(o.batches * outer * o.pitch * es + 255) / 256 * 256;
  }
  return o;
}

void plan(int64_t rows, int64_t inner, int64_t cols, int64_t batch, int64_t left_stride, int64_t right_stride,
          int ta, int tb, int a_dtype, int b_dtype, bool bf16, const void* a, const void* b, Operand* pa,
          Operand* pb) {
  *pa = ta ? plan_operand(a, a_dtype, bf16, inner, rows, batch, left_stride)
           : plan_operand(a, a_dtype, bf16, rows, inner, batch, left_stride);
  *pb = tb ? plan_operand(b, b_dtype, bf16, cols, inner, batch, right_stride)
           : plan_operand(b, b_dtype, bf16, inner, cols, batch, right_stride);
}

// A re-laid-out row must fit the kernel's 32-bit chunk indices (any row of
// a valid operand does); larger operands take several launches.
bool prepare_fits(const Operand& o) { return o.pitch < (1ll << 31) && o.inner < (1ll << 32); }

// The re-layout launches of one operand: rows [base, base + r) per launch,
// r * pitch / E below 2^31 chunks.
int prepare_launches(const Operand& o, bool bf16) {
  const int64_t rows = o.batches * o.outer, per_row = o.pitch / (bf16 ? 8 : 4);
  const int64_t step = std::max<int64_t>(1, ((1ll << 31) - 1) / per_row);
  return (int)((rows + step - 1) / step);
}

PrepareArgs prepare_args(const Operand& o, bool bf16, char* ws, int64_t base, uint32_t rows) {
  PrepareArgs a;
  a.src = o.ptr;
  a.dst = ws;
  a.row_base = base;
  a.outer = o.outer;
  a.stride = o.src_stride;
  a.rows = rows;
  a.inner = (uint32_t)o.inner;
  a.pitch = (uint32_t)o.pitch;
  (void)bf16;
  return a;
}

void launch_prepare(Operand& o, int src_dtype, bool bf16, char* ws, hipStream_t stream) {
  const int64_t rows = o.batches * o.outer, per_row = o.pitch / (bf16 ? 8 : 4);
  const int64_t step = std::max<int64_t>(1, ((1ll << 31) - 1) / per_row);  // rows per launch
  for (int64_t base = 0; base < rows; base += step) {
    const uint32_t r = (uint32_t)std::min<int64_t>(step, rows - base);
    const dim3 grid((unsigned)(((int64_t)r * per_row + 256 * PREP_CHUNKS - 1) / (256 * PREP_CHUNKS)));
    const PrepareArgs a = prepare_args(o, bf16, ws, base, r);
    if (src_dtype == QA_BF16 && bf16) hipLaunchKernelGGL((prepare_operand<true, true>), grid, dim3(256), 0, stream, a);
    else if (bf16) hipLaunchKernelGGL((prepare_operand<false, true>), grid, dim3(256), 0, stream, a);
    else if (src_dtype == QA_BF16) hipLaunchKernelGGL((prepare_operand<true, false>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((prepare_operand<false, false>), grid, dim3(256), 0, stream, a);
  }
  o.ptr = ws;
}

// The column remainder alone (B used in place: its source dtype is the
// compute type).
void launch_remainder(const RemainderArgs& r, bool bf16, bool kb, hipStream_t stream) {
  const dim3 grid((unsigned)((r.M + RBLOCK - 1) / RBLOCK)), block(64 * RWAVES);
  if (bf16 && kb) hipLaunchKernelGGL((remainder_columns<true, true, true>), grid, block, 0, stream, r);
  else if (bf16) hipLaunchKernelGGL((remainder_columns<true, true, false>), grid, block, 0, stream, r);
  else if (kb) hipLaunchKernelGGL((remainder_columns<false, false, true>), grid, block, 0, stream, r);
  else hipLaunchKernelGGL((remainder_columns<false, false, false>), grid, block, 0, stream, r);
}

// B's re-layout (one launch) with the column remainder in the same grid.
void launch_prepare_remainder(Operand& o, int src_dtype, bool bf16, bool kb, char* ws, const RemainderArgs& r,
                              hipStream_t stream) {
  const int64_t rows = o.batches * o.outer, per_row = o.pitch / (bf16 ? 8 : 4);
  const unsigned rem = (unsigned)((r.M + RBLOCK - 1) / RBLOCK);
  const dim3 grid((unsigned)(rem + (rows * per_row + 256 * PREP_CHUNKS - 1) / (256 * PREP_CHUNKS)));
  const PrepareArgs a = prepare_args(o, bf16, ws, 0, (uint32_t)rows);
  const bool sb = src_dtype == QA_BF16;
  if (sb && bf16 && kb) hipLaunchKernelGGL((prepare_remainder<true, true, true>), grid, dim3(256), 0, stream, a, r, rem);
  else if (sb && bf16) hipLaunchKernelGGL((prepare_remainder<true, true, false>), grid, dim3(256), 0, stream, a, r, rem);
  else if (bf16 && kb) hipLaunchKernelGGL((prepare_remainder<false, true, true>), grid, dim3(256), 0, stream, a, r, rem);
  else if (bf16) hipLaunchKernelGGL((prepare_remainder<false, true, false>), grid, dim3(256), 0, stream, a, r, rem);
  else if (sb && kb) hipLaunchKernelGGL((prepare_remainder<true, false, true>), grid, dim3(256), 0, stream, a, r, rem);
  else if (sb) hipLaunchKernelGGL((prepare_remainder<true, false, false>), grid, dim3(256), 0, stream, a, r, rem);
  else if (kb) hipLaunchKernelGGL((prepare_remainder<false, false, true>), grid, dim3(256), 0, stream, a, r, rem);
  else hipLaunchKernelGGL((prepare_remainder<false, false, false>), grid, dim3(256), 0, stream, a, r, rem);
  o.ptr = ws;
}

// Short-K strip launch (tile R): the call's rows are K-major for both
// operands (NT), K <= 64, bf16 output without accumulation, output rows
// 16-byte aligned and N a multiple of 16 (every 16-byte store is inside or
// wholly outside a row).  Each workgroup
// sweeps `strip` 128-column chunks; strips shrink (halving) until the grid
// holds at least 16 rounds of the two workgroups a CU runs at once.  Config
// 3's score product (128 x 2048 x 2048, K 64): 208 us with one chunk per
// workgroup, 181-185 us with 2, 4 or 8 (the rule gives 4), 200 us with 16.
// The two-slot ring (50 KiB of LDS) under a 168-register cap fits three
// workgroups per CU instead of two: 179-183 -> 166-170 us alone, the bmm
// sequence 789 -> 772 us, bit-identical.
bool short_fits(const GemmArgs& p, bool bf16, bool ta, bool tb) {
  return bf16 && !ta && tb && p.out_bf16 && !p.accumulate && p.K > 0 && p.K <= 64 && p.N % 16 == 0 &&
         p.vec_c == 2 && p.ldc * 128 * 2 < (1ll << 31);
}
hipError_t launch_short(const GemmArgs& p, hipStream_t stream) {
  ShortArgs s = {};
  s.a = (const bf16_t*)p.a;
  s.b = (const bf16_t*)p.b;
  s.out = p.out;
  s.M = p.M;
  s.N = p.N;
  s.K = p.K;
  s.lda = p.lda;
  s.ldb = p.ldb;
  s.ldc = p.ldc;
  s.sa = p.sa;
  s.sb = p.sb;
  s.sc = p.sc;
  s.batch = p.batch;
  s.alpha = p.alpha;
  s.tiles_m = (int)((p.M + 127) / 128);
  s.chunks = (int)((p.N + 127) / 128);
  int strip = s.chunks;
  typedef ShortKernel<2> Kern;
  const int64_t slots = Kern::MIN_BLOCKS * cu_count();
  while (strip > 1 && p.batch * s.tiles_m * ((s.chunks + strip - 1) / strip) < 16 * slots) strip = (strip + 1) / 2;
  s.strip_chunks = strip;
  s.strips = (s.chunks + strip - 1) / strip;
  if (p.batch * s.tiles_m * s.strips > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(short_entry<Kern>, dim3((unsigned)(p.batch * s.tiles_m * s.strips)), dim3(Kern::NT), 0, stream,
                     s);
  return hipGetLastError();
}

// 4-wide output stores need 4 | ldc, 4 | batch stride and an aligned base.
// 2: every output row starts 16-byte aligned for both element sizes;
// 1: 16-byte aligned fp32 rows / 8-byte aligned bf16 rows; 0: neither.
int vec_out(const void* p, int64_t ldc, int64_t stride) {
  if ((uintptr_t)p % 16 != 0) return 0;
  if (ldc % 8 == 0 && stride % 8 == 0) return 2;
  return (ldc % 4 == 0 && stride % 4 == 0) ? 1 : 0;
}

// One launch of a plain product over output columns [c0, c0 + n): its tile,
// K chunks and fp32 partial bytes.
struct Window {
  int64_t c0, n;
  Tile tile;
  int splits;
  int64_t chunk;
  size_t partial;
  bool rows_kernel;  // remainder_columns instead of a tile
};

// The launches of a plain product: one window over every column or, with a
// column remainder (column_split), the large-tile columns and the rest: up
// to 8 columns of a K-major A on remainder_columns (one launch, no partial
// sums), wider remainders on the thin tile.
int plan_windows(int64_t rows, int64_t inner, int64_t cols, int64_t batch, bool bf16, int transpose_left,
                 Window (&w)[2]) {
  const int64_t main_cols = inner > 0 ? column_split(rows, cols, inner, batch, bf16) : 0;
  const int count = main_cols ? 2 : 1;
  for (int i = 0; i < count; i++) {
    Window& x = w[i];
    x.c0 = i == 0 ? 0 : main_cols;
    x.n = count == 1 ? cols : i == 0 ? main_cols : cols - main_cols;
    x.rows_kernel = i == 1 && x.n <= 8 && !transpose_left;
    x.tile = choose_tile(rows, x.n, inner, batch, bf16);
    x.chunk = 0;
    x.splits = inner > 0 && !x.rows_kernel ? choose_split(rows, x.n, inner, batch, &x.tile, bf16, &x.chunk) : 1;
    x.partial = x.splits > 1 ? split_bytes(rows, x.n, batch, x.splits) : 0;

  }
  return count;
}

}  // namespace

extern "C" {

size_t qutai_amd_gemm_workspace_size(int64_t rows, int64_t inner, int64_t cols, int64_t batch,
                                     int64_t left_stride, int64_t right_stride, int transpose_left,
                                     int transpose_right, int a_dtype, int b_dtype, int bf16_compute) {
  if (a_dtype == QA_F64 || b_dtype == QA_F64 || batch <= 0 || rows * cols == 0 || inner == 0) return 0;
  bool bf16 = bf16_compute || a_dtype == QA_BF16 || b_dtype == QA_BF16;
  Operand pa, pb;
  // 256-byte aligned pointers: only dtype and row alignment decide
  plan(rows, inner, cols, batch, left_stride, right_stride, transpose_left, transpose_right, a_dtype, b_dtype, bf16,
       (const void*)256, (const void*)256, &pa, &pb);
  Window w[2];
  const int count = plan_windows(rows, inner, cols, batch, bf16, transpose_left, w);
  size_t partial = 0;
  for (int i = 0; i < count; i++) partial += w[i].partial;
  if (!pa.copy && !pb.copy && !partial) return 0;
  return (pa.copy ? pa.bytes : 0) + (pb.copy ? pb.bytes : 0) + partial + 256;
}

int qutai_amd_gemm(const void* a, const void* b, void* out, int64_t rows, int64_t inner, int64_t cols,
                   int64_t batch, int64_t left_stride, int64_t right_stride, int transpose_left,
                   int transpose_right, int a_dtype, int b_dtype, int out_dtype, int accumulate,
                   int bf16_compute, void* workspace, size_t workspace_bytes, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (rows < 0 || inner < 0 || cols < 0 || batch < 0 || left_stride < 0 || right_stride < 0) return QA_EINVAL;
  bool f64 = a_dtype == QA_F64 || b_dtype == QA_F64;
  for (int d : {a_dtype, b_dtype})
    if (d != QA_F32 && d != QA_BF16 && d != QA_F64) return QA_EINVAL;
  if (f64 && (a_dtype != b_dtype || out_dtype != QA_F64)) return QA_EINVAL;
  if (!f64 && out_dtype != QA_F32 && out_dtype != QA_BF16) return QA_EINVAL;
  int64_t size = batch * rows * cols;
  if (size == 0) return QA_OK;
  if (!out) return QA_EINVAL;
  if (inner > 0 && (!a || !b)) return QA_EINVAL;
  if (f64) {
    int64_t tiles_m = (rows + 31) / 32, tiles_n = (cols + 31) / 32;
    int64_t blocks = tiles_m * tiles_n * batch;
    if (blocks > 0x7fffffff) return QA_EINVAL;
    hipLaunchKernelGGL(gemm_f64, dim3((unsigned)blocks), dim3(256), 0, stream, (const double*)a, (const double*)b,
                       (double*)out, rows, inner, cols, left_stride, right_stride, transpose_left, transpose_right,
                       accumulate, tiles_n, tiles_m);
    return (int)hipGetLastError();
  }
  bool bf16 = bf16_compute || a_dtype == QA_BF16 || b_dtype == QA_BF16;
  Operand pa, pb;
  plan(rows, inner, cols, batch, left_stride, right_stride, transpose_left, transpose_right, a_dtype, b_dtype, bf16,
       a, b, &pa, &pb);
  Window w[2];
  const int count = plan_windows(rows, inner, cols, batch, bf16, transpose_left, w);
  size_t partial = 0;
  for (int i = 0; i < count; i++) partial += w[i].partial;
  char* part = nullptr;
  // the column remainder's arguments: A as planned (re-laid out before it
  // runs), B's r columns from column c0 of `b_ptr` (row pitch ldb_src)
  const int osize_ = out_dtype == QA_BF16 ? 2 : 4;
  auto remainder_args = [&](const void* a_ptr, const void* b_ptr, const Window& x, int64_t ldb_src) {
    RemainderArgs r = {};
    r.a = a_ptr;
    r.b = b_ptr;
    r.out = (char*)out + x.c0 * osize_;
    r.M = rows;
    r.K = inner;
    r.lda = pa.ld;
    r.ldb = ldb_src;
    r.ldc = cols;
    r.col = x.c0;
    r.r = (int)x.n;
    r.out_bf16 = out_dtype == QA_BF16 ? 1 : 0;
    r.accumulate = accumulate ? 1 : 0;
    return r;
  };
  bool fused_remainder = false;
  if (inner > 0 && ((pa.copy && !prepare_fits(pa)) || (pb.copy && !prepare_fits(pb)))) return QA_EINVAL;
  if (inner > 0 && (pa.copy || pb.copy || partial)) {
    size_t need = (pa.copy ? pa.bytes : 0) + (pb.copy ? pb.bytes : 0) + partial + 256;
    if (workspace == nullptr || workspace_bytes < need) return QA_EWORKSPACE;
    char* ws = (char*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
    if (pa.copy) {
      launch_prepare(pa, a_dtype, bf16, ws, stream);
      ws += pa.bytes;
    }
    if (pb.copy) {
      // B's re-layout shares its launch with a column remainder (which reads
      // B at its source pitch and dtype) when it takes one launch
      if (count == 2 && w[1].rows_kernel && prepare_launches(pb, bf16) == 1) {
        fused_remainder = true;
        launch_prepare_remainder(pb, b_dtype, bf16, transpose_right, ws,
                                 remainder_args(pa.ptr, b, w[1], transpose_right ? inner : cols), stream);
      } else {
        launch_prepare(pb, b_dtype, bf16, ws, stream);
      }
      ws += pb.bytes;
    }
    if (partial) part = ws;
  }
  GemmArgs p = {};
  p.a = pa.ptr;
  p.b = pb.ptr;
  p.out = out;
  p.M = rows;
  p.N = cols;
  p.K = inner;
  p.lda = pa.ld;
  p.ldb = pb.ld;
  p.ldc = cols;
  p.sa = pa.stride;
  p.sb = pb.stride;
  p.sc = rows * cols;
  p.batch = batch;
  p.accumulate = accumulate ? 1 : 0;
  p.out_bf16 = out_dtype == QA_BF16;
  p.vec_c = vec_out(out, p.ldc, p.sc);
  p.alpha = 1.0f;
  // buffer descriptors address at most 2^31 bytes per K step
  int64_t es = bf16 ? 2 : 4;
  if ((p.lda * 256 * es) >= (1ll << 31) || (p.ldb * 256 * es) >= (1ll << 31)) return QA_EINVAL;
  const int osize = out_dtype == QA_BF16 ? 2 : 4;
  for (int i = 0; i < count; i++) {
    const Window& x = w[i];
    GemmArgs q = p;
    // the window's columns: B's rows (K-major) or columns from c0, out's
    // columns from c0 at the full row pitch
    q.N = x.n;
    q.b = (const char*)pb.ptr + x.c0 * (transpose_right ? pb.ld : 1) * es;
    char* window_out = (char*)out + x.c0 * osize;
    q.out = window_out;
    q.vec_c = vec_out(window_out, q.ldc, q.sc);
    float* window_part = nullptr;
    if (x.partial && !x.rows_kernel) {
      // fp32 partials of each K chunk ([rows][n] each), then the ordered sum
      window_part = (float*)part;
      part += x.partial;
      q.out = window_part;
      q.ldc = x.n;
      q.sc = rows * x.n;
      q.k_split = x.splits;
      q.k_chunk = x.chunk;
      q.batch = batch * x.splits;
      q.accumulate = 0;
      q.out_bf16 = 0;
      q.vec_c = vec_out(window_part, q.ldc, q.sc);
    }
    if (x.rows_kernel) {
      // the last r columns: done with B's re-layout, or one launch of their own
      if (!fused_remainder) {
        launch_remainder(remainder_args(q.a, pb.ptr, x, pb.ld), bf16, transpose_right, stream);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return (int)err;
      }
      continue;
    }
    if (!window_part && count == 1 && ((x.tile == TILE_S2 && forced_tile() < 0) || x.tile == TILE_R) &&
        short_fits(q, bf16, transpose_left, transpose_right))
      return (int)launch_short(q, stream);
    hipError_t err = bf16 ? launch_mma<false>(x.tile, transpose_left, transpose_right, q, stream)
                          : launch_mma<true>(x.tile, transpose_left, transpose_right, q, stream);
    if (err != hipSuccess) return (int)err;
    if (!window_part) continue;
    const int64_t total = batch * rows * x.n;
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 1 << 20);
    hipLaunchKernelGGL(splitk_reduce, dim3(blocks), dim3(256), 0, stream, (const float*)window_part,
                       (void*)window_out, rows * x.n, total, x.splits, accumulate ? 1 : 0,
                       out_dtype == QA_BF16 ? 1 : 0, x.n, cols);
    err = hipGetLastError();
    if (err != hipSuccess) return (int)err;
  }
  return QA_OK;
}

int qutai_amd_gemm_grouped(const void* a, const void* b, void* out, const int64_t* offsets, int groups,
                           int64_t max_rows, int64_t inner, int64_t cols, int64_t expert_stride,
                           int transpose_right, int dtype, int out_dtype, int accumulate, const int64_t* gather,
                           int64_t source_rows, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (groups <= 0 || max_rows < 0 || inner < 0 || cols < 0 || expert_stride < 0) return QA_EINVAL;
  if (dtype != QA_BF16 && dtype != QA_F32) return QA_EINVAL;
  if (out_dtype != QA_F32 && out_dtype != QA_BF16) return QA_EINVAL;
  if (!offsets || !out) return QA_EINVAL;
  if (max_rows == 0 || cols == 0) return QA_OK;
  GemmArgs p = {};
  p.a = a;
  p.b = b;
  p.out = out;
  p.M = max_rows;
  p.N = cols;
  p.K = inner;
  p.lda = inner;
  p.ldb = transpose_right ? inner : cols;
  p.ldc = cols;
  p.sb = expert_stride;
  p.batch = 1;
  p.accumulate = accumulate ? 1 : 0;
  p.out_bf16 = out_dtype == QA_BF16;
  int64_t E = dtype == QA_BF16 ? 8 : 4;
  if ((uintptr_t)a % 16 || (uintptr_t)b % 16 || inner % E || p.ldb % E || expert_stride % E) return QA_EINVAL;
  // a 256-row tile's operand range must fit the 31-bit buffer descriptor
  const int64_t es = dtype == QA_BF16 ? 2 : 4;
  if ((p.lda * 256 * es) >= (1ll << 31) || (p.ldb * 256 * es) >= (1ll << 31)) return QA_EINVAL;
  p.vec_c = vec_out(out, p.ldc, 0);
  p.offsets = offsets;
  p.groups = groups;
  p.alpha = 1.0f;
  if (gather) {
    // row offsets into a are 32-bit byte offsets of one buffer descriptor
    if (source_rows < 0 || source_rows * inner * es >= (1ll << 31)) return QA_EINVAL;
    p.a_rows = gather;
    p.a_bytes = source_rows * inner * es;
  }
  Tile tile = grouped_tile(max_rows, cols, groups, dtype == QA_BF16);
  if (gather && tile == TILE_L8R) tile = TILE_L8D2;  // gathered rows need the DMA ring
  const int bm = tile_rows(tile);
  p.tiles_m = (int)((max_rows + bm - 1) / bm + groups);
  bool f32 = dtype == QA_F32;
  hipError_t err = f32 ? launch_mma<true>(tile, false, transpose_right, p, stream)
                       : launch_mma<false>(tile, false, transpose_right, p, stream);
  return (int)err;
}

int qutai_amd_gemm_grouped_pair(const void* a, const void* a_tail, const void* b, const void* b_tail, void* out,
                                const int64_t* offsets, int groups, int64_t max_rows, int64_t inner, int64_t cols,
                                int64_t expert_stride, int transpose_right, int dtype, int out_dtype, int accumulate,
                                void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (groups <= 0 || max_rows < 0 || inner < 0 || cols < 0 || expert_stride < 0) return QA_EINVAL;
  if (dtype != QA_BF16 && dtype != QA_F32) return QA_EINVAL;
  if (out_dtype != QA_F32 && out_dtype != QA_BF16) return QA_EINVAL;
  if (!offsets || !out) return QA_EINVAL;
  // the join must fall on a K step of every tile configuration (64 / 32)
  if (inner % 64) return QA_EINVAL;
  if (max_rows == 0 || cols == 0) return QA_OK;
  if (inner == 0) return QA_EINVAL;
  GemmArgs p = {};
  p.a = a;
  p.b = b;
  p.a_tail = a_tail;
  p.b_tail = b_tail;
  p.k_head = inner;
  p.out = out;
  p.M = max_rows;
  p.N = cols;
  p.K = 2 * inner;
  p.lda = inner;
  p.ldb = transpose_right ? inner : cols;
  p.ldc = cols;
  p.sb = expert_stride;
  p.batch = 1;
  p.accumulate = accumulate ? 1 : 0;
  p.out_bf16 = out_dtype == QA_BF16;
  const int64_t E = dtype == QA_BF16 ? 8 : 4;
  for (const void* q : {a, a_tail, b, b_tail})
    if (!q || (uintptr_t)q % 16) return QA_EINVAL;
  if (p.ldb % E || expert_stride % E) return QA_EINVAL;
  const int64_t es = dtype == QA_BF16 ? 2 : 4;
  if ((p.lda * 256 * es) >= (1ll << 31) || (p.ldb * 256 * es) >= (1ll << 31)) return QA_EINVAL;
  p.vec_c = vec_out(out, p.ldc, 0);
  p.offsets = offsets;
  p.groups = groups;
  p.alpha = 1.0f;
  Tile tile = grouped_tile(max_rows, cols, groups, dtype == QA_BF16);
  const int bm = tile_rows(tile);
  p.tiles_m = (int)((max_rows + bm - 1) / bm + groups);
  hipError_t err = dtype == QA_F32 ? launch_mma<true>(tile, false, transpose_right, p, stream)
                                   : launch_mma<false>(tile, false, transpose_right, p, stream);
  return (int)err;
}

int qutai_amd_gemm_swiglu(const void* a, const void* w_gate, const void* w_up, void* out, void* gate_out,
                          void* up_out, const int64_t* offsets, int groups, int64_t rows, int64_t inner,
                          int64_t hidden, int64_t expert_stride, int dtype, const int64_t* gather,
                          int64_t source_rows, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (rows < 0 || inner < 0 || hidden < 0 || expert_stride < 0 || (offsets && groups <= 0)) return QA_EINVAL;
  if (dtype != QA_BF16) return QA_EINVAL;
  if (!out || (rows > 0 && hidden > 0 && (!a || !w_gate || !w_up))) return QA_EINVAL;
  if (rows == 0 || hidden == 0) return QA_OK;
  if ((uintptr_t)a % 16 || (uintptr_t)w_gate % 16 || (uintptr_t)w_up % 16 || inner % 8 || expert_stride % 8)
    return QA_EINVAL;
  for (void* o : {out, gate_out, up_out})
    if (o && (uintptr_t)o % 16) return QA_EINVAL;
  GemmArgs p = {};
  p.a = a;
  p.b = w_gate;
  p.b2 = w_up;
  p.out = out;
  p.gate_out = gate_out;
  p.up_out = up_out;
  p.M = rows;
  p.N = hidden;
  p.K = inner;
  p.lda = inner;
  p.ldb = inner;
  p.ldc = hidden;
  p.sb = offsets ? expert_stride : 0;
  p.sc = rows * hidden;
  p.batch = 1;
  p.out_bf16 = 1;
  p.vec_c = vec_out(out, p.ldc, 0);
  p.alpha = 1.0f;
  if ((p.lda * 256 * 2) >= (1ll << 31)) return QA_EINVAL;
  if (gather) {
    if (!offsets || source_rows < 0 || source_rows * inner * 2 >= (1ll << 31)) return QA_EINVAL;
    p.a_rows = gather;
    p.a_bytes = source_rows * inner * 2;
  }
  if (offsets) {
    p.offsets = offsets;
    p.groups = groups;
    p.tiles_m = (int)((rows + 255) / 256 + groups);
  }
  return (int)launch_cfg<false, false, true, 256, 256, 2, 4, 64, 2, true, true>(p, stream);
}

int qutai_amd_gemm_grouped_k(const void* a, const void* b, void* out, const int64_t* offsets, int groups, int64_t rows,
                             int64_t cols, int64_t total_k, int dtype, int out_dtype, int accumulate,
                             const int64_t* gather, int64_t source_rows, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (groups <= 0 || rows < 0 || cols < 0 || total_k < 0) return QA_EINVAL;
  if (dtype != QA_BF16 && dtype != QA_F32) return QA_EINVAL;
  if (out_dtype != QA_F32 && out_dtype != QA_BF16) return QA_EINVAL;
  if (!offsets || !out) return QA_EINVAL;
  if (rows == 0 || cols == 0) return QA_OK;
  const int64_t E = dtype == QA_BF16 ? 8 : 4;
  if ((uintptr_t)a % 16 || (uintptr_t)b % 16 || rows % E || cols % E) return QA_EINVAL;
  GemmArgs p = {};
  p.a = a;
  p.b = b;
  p.out = out;
  p.M = rows;
  p.N = cols;
  p.K = total_k;
  p.lda = rows;  // A stored [K][rows]: out_g = A_g^T B_g
  p.ldb = cols;  // B stored [K][cols]
  p.ldc = cols;
  p.sc = rows * cols;
  p.batch = groups;
  p.accumulate = accumulate ? 1 : 0;
  p.out_bf16 = out_dtype == QA_BF16;
  p.vec_c = vec_out(out, p.ldc, p.sc);
  p.offsets = offsets;
  p.group_k = 1;
  p.alpha = 1.0f;
  int64_t es = dtype == QA_BF16 ? 2 : 4;
  if ((p.lda * 256 * es) >= (1ll << 31) || (p.ldb * 256 * es) >= (1ll << 31)) return QA_EINVAL;
  Tile tile = choose_tile(rows, cols, total_k / groups + 1, groups, dtype == QA_BF16);
  if (gather) {
    // row offsets into b are 32-bit byte offsets of one buffer descriptor
    if (source_rows < 0 || source_rows * cols * es >= (1ll << 31)) return QA_EINVAL;
    p.b_rows = gather;
    p.b_bytes = source_rows * cols * es;
    return (int)(dtype == QA_F32 ? launch_gathered_k<true>(tile, p, stream)
                                 : launch_gathered_k<false>(tile, p, stream));
  }
  hipError_t err = dtype == QA_F32 ? launch_mma<true>(tile, true, false, p, stream)
                                   : launch_mma<false>(tile, true, false, p, stream);
  return (int)err;
}

}  // extern "C"
