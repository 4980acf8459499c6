// Short-K bf16 NT product for gfx950:
//   C[b][m][n] (+)= alpha * sum_{k < K} A[b][m][k] * B[b][n][k],   K <= 64,
// the shape of the attention score product S = Q K^T (config 3: K = 64, the
// head size; src/qutai/backends/cuda.py:346-355 runs it as a batched NT gemm).
//
// Such a product writes one output element per 2K FLOPs, so it is bound by
// the output stream and by how fast short-lived tiles can be fed.  One
// workgroup keeps a 128-row block of A in registers and sweeps its strip of
// N: every strips-th 128-column chunk (strip, strip + strips, ...), so the
// workgroups of a row block write neighbouring chunks of the same rows at
// the same time:
//  * the B chunks move HBM/L2 -> LDS with direct-to-LDS buffer loads into a
//    SLOTS-deep ring, SLOTS - 1 chunks ahead of the MFMAs (two slots: three
//    workgroups fit per CU, which keeps more stores in flight);
//  * the MFMAs compute the transposed block (B rows as the first operand), so
//    a lane's accumulators hold four consecutive columns of one row; one
//    gfx950 lane-half swap (v_permlane32_swap) gives every lane eight
//    consecutive bf16 columns, which go through a small per-wave LDS stage
//    and leave as 128-byte row segments: streaming (nontemporal) stores of
//    whole lines (partial-line streaming stores measured 4x slower);
//  * out-of-range rows and columns get an out-of-range buffer offset, so every
//    store instruction is issued by every wave: the number of memory operations
//    issued after each chunk's copies is fixed, and the wait for that chunk is
//    an exact `s_waitcnt vmcnt(n)` that never waits for the stores (vector
//    memory operations complete in issue order on gfx9).
// The K sum runs in the order of the other GEMM tiles (16-wide MFMA steps from
// k = 0, fp32) and the epilogue rounds like theirs (alpha, one rounding), so
// this tile gives the same bits as the 128x128 / 256x256 tiles.  bf16 output
// without accumulation only (the score product); other calls take those tiles.
#pragma once
#include "gemm_kernel.h"

namespace qa {

struct ShortArgs {
  const bf16_t* a;  // [batch][M][lda] K-major rows, 16-byte aligned
  const bf16_t* b;  // [batch][N][ldb]
  void* out;        // [batch][M][ldc], 16-byte aligned rows
  int64_t M, N, K, lda, ldb, ldc, sa, sb, sc;
  int64_t batch;
  int tiles_m, strips, chunks, strip_chunks;  // grid = batch * tiles_m * strips
  float alpha;
};

template <int SLOTS>
struct ShortKernel {
  static constexpr int BM = 128, BN = 128, BK = 64, NW = 4, NT = 64 * NW;
  typedef OperandTile<false, true, 128, 64> Tile;  // [128][64] bf16, swizzled 16-byte chunks
  static constexpr int TILE_BYTES = BM * BK * 2;   // 16 KB
  // output stage: 32 rows x 64 bf16 per wave, rows padded to 144 bytes; it
  // reuses the A block's LDS once A is in registers
  static constexpr int SP = 144, STAGE_BYTES = NW * 32 * SP;
  static constexpr int HEAD = STAGE_BYTES > TILE_BYTES ? STAGE_BYTES : TILE_BYTES;
  static constexpr int LDS_BYTES = HEAD + SLOTS * TILE_BYTES;
  static constexpr int J = Tile::CHUNKS / NT;      // copy instructions per wave and tile (4)
  static constexpr int OPS = 8;                    // stores per wave and chunk
  static constexpr uint32_t OOB = 0x80000000u;
  static_assert(J == 4 && SLOTS >= 2 && SLOTS <= 3, "shape");
  // workgroups per CU the launch bounds ask for: with two slots the LDS
  // (50 KiB) and a 168-register cap fit three (12 waves per CU)
  static constexpr int MIN_BLOCKS = SLOTS == 2 ? 3 : 2;

  template <int N>
  __device__ static __forceinline__ void wait_vm() {
    wait_vmcnt<(N < 63 ? N : 63)>();
  }
  __device__ static __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

  // lane's fragment of rows [row, row + 32), k = 16 s + 8 (lane >> 5) + [0, 8)
  __device__ static __forceinline__ bf16x8 frag(const bf16_t* t, int row, int s, int lane) {
    const int r = row + (lane & 31), c = 2 * s + (lane >> 5);
    return *reinterpret_cast<const bf16x8*>(t + r * BK + ((c ^ swz_k<8>(r)) * 8));
  }

  __device__ static __forceinline__ void run(const ShortArgs& p, char* smem) {
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform32(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;  // 64 x 64 per wave
    const int total = p.batch * p.tiles_m * p.strips;
    const int pid = uniform32(xcd_remap((int)blockIdx.x, total));
    const int strip = pid % p.strips, tm = (pid / p.strips) % p.tiles_m;
    const int64_t bz = pid / (p.strips * p.tiles_m);
    const int64_t row0 = (int64_t)tm * BM;
    // this strip's chunks are strip, strip + strips, ...: the workgroups of
    // one row block (consecutive ids, one XCD) write neighbouring 128-column
    // chunks of the same rows at the same time
    const int nc = uniform32((p.chunks - strip + p.strips - 1) / p.strips);
    const int64_t K = p.K;

    const bf16_t* A = uniform_ptr(p.a + bz * p.sa + row0 * p.lda);
    const bf16_t* B = uniform_ptr(p.b + bz * p.sb);
    char* lds_a = smem;
    char* ring = smem + HEAD;
    char* stage = smem + wave * 32 * SP;

    // this lane's (row, chunk) of each copy instruction
    int cr[J], cc[J];
#pragma unroll
    for (int j = 0; j < J; j++) Tile::coords((j * NW + wave) * 64 + lane, cr[j], cc[j]);
    auto copy = [&](const bf16_t* base, int64_t ld, int64_t rows_left, char* dst) {
      const u32x4 d = lds_rsrc(base, (int64_t)BM * ld * 2);
#pragma unroll
      for (int j = 0; j < J; j++) {
        const bool ok = cr[j] < rows_left && cc[j] * 8 < K;
        lds_load16(d, dst + (j * NW + wave) * 1024, ok ? (uint32_t)((cr[j] * ld + cc[j] * 8) * 2) : OOB);
      }
    };
    auto copy_b = [&](int c) {  // chunk c of the strip into its ring slot
      const int64_t n0 = (int64_t)(strip + c * p.strips) * BN;
      copy(uniform_ptr(B + n0 * p.ldb), p.ldb, p.N - n0, ring + (c % SLOTS) * TILE_BYTES);
    };

    // output rows of this lane: row0 + wm*64 + fm*32 + (lane & 31); the
    // descriptor covers the tile's rows that exist
    constexpr int ES = 2;
    const int64_t rows_here = p.M - row0 < BM ? p.M - row0 : BM;
    char* obase = uniform_ptr(reinterpret_cast<char*>(p.out) + (bz * p.sc + row0 * p.ldc) * ES);
    const int64_t orange = rows_here * p.ldc * ES;
    const __amdgpu_buffer_rsrc_t od =
        __builtin_amdgcn_make_buffer_rsrc(obase, 0, (int)(orange > 0x7ffffff0 ? 0x7ffffff0 : orange), 0x00020000);

    // prologue: A block, then the first SLOTS - 1 chunks of B
    copy(A, p.lda, p.M - row0, lds_a);
#pragma unroll
    for (int c = 0; c < SLOTS - 1; c++)
      if (c < nc) copy_b(c);
    if (SLOTS == 3 && nc > 1) wait_vm<J>();
    else wait_vm<0>();
    barrier();
    bf16x8 fa[2][4];  // A fragments: 2 row blocks x 4 k-steps, for the whole strip
#pragma unroll
    for (int fm = 0; fm < 2; fm++)
#pragma unroll
      for (int s = 0; s < 4; s++) fa[fm][s] = frag(reinterpret_cast<const bf16_t*>(lds_a), wm * 64 + fm * 32, s, lane);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the A fragments are in registers
    barrier();                           // before any wave's output stage overwrites the A block

    for (int c = 0; c < nc; c++) {
      const bool ahead = c + SLOTS - 1 < nc;
      if (ahead) copy_b(c + SLOTS - 1);  // into the slot of chunk c - 1, read by every wave
      const bf16_t* sb = reinterpret_cast<const bf16_t*>(ring + (c % SLOTS) * TILE_BYTES);
      f32x16 acc[2][2];
#pragma unroll
      for (int fm = 0; fm < 2; fm++)
#pragma unroll
        for (int fn = 0; fn < 2; fn++)
#pragma unroll
          for (int e = 0; e < 16; e++) acc[fm][fn][e] = 0.f;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        bf16x8 fb[2];
#pragma unroll
        for (int fn = 0; fn < 2; fn++) fb[fn] = frag(sb, wn * 64 + fn * 32, s, lane);
#pragma unroll
        for (int fm = 0; fm < 2; fm++)
#pragma unroll
          for (int fn = 0; fn < 2; fn++)
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[fn], fa[fm][s], acc[fm][fn], 0, 0, 0);
      }
      // acc[fm][fn][e]: row wm*64 + fm*32 + (lane & 31), column
      // wn*64 + fn*32 + 8 (e >> 2) + 4 (lane >> 5) + (e & 3) of the chunk.
      // One 32-row block at a time: the lane-half swap gives each lane 8
      // consecutive columns (16 bytes), staged in LDS and read back as whole
      // 128-byte row segments, so every streaming store writes full lines.
      const int64_t n0 = (int64_t)(strip + c * p.strips) * BN + wn * 64;
#pragma unroll
      for (int fm = 0; fm < 2; fm++) {
#pragma unroll
        for (int fn = 0; fn < 2; fn++) {
          const f32x16 v = acc[fm][fn] * p.alpha;
#pragma unroll
          for (int h = 0; h < 2; h++) {
            // v[8h..8h+3]: columns 0-3 of group 2h in lanes < 32, 4-7 in
            // lanes >= 32; v[8h+4..8h+7]: group 2h + 1 likewise.  After the
            // swap a lane < 32 holds columns 0-7 of group 2h, a lane >= 32
            // columns 0-7 of group 2h + 1.
            auto lo = __builtin_amdgcn_permlane32_swap(pack_bf16x2(v[8 * h], v[8 * h + 1]),
                                                       pack_bf16x2(v[8 * h + 4], v[8 * h + 5]), false, false);
            auto hi = __builtin_amdgcn_permlane32_swap(pack_bf16x2(v[8 * h + 2], v[8 * h + 3]),
                                                       pack_bf16x2(v[8 * h + 6], v[8 * h + 7]), false, false);
            const int col = fn * 32 + 16 * h + 8 * (lane >> 5);
            *reinterpret_cast<u32x4*>(stage + (lane & 31) * SP + col * 2) = u32x4{lo[0], hi[0], lo[1], hi[1]};
          }
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int it = 0; it < 4; it++) {
          const int idx = it * 64 + lane, r = idx >> 3, q = idx & 7;
          const u32x4 w = *reinterpret_cast<const u32x4*>(stage + r * SP + q * 16);
          const int64_t col = n0 + 8 * q;
          const uint32_t off =
              col < p.N ? (uint32_t)(((int64_t)(wm * 64 + fm * 32 + r) * p.ldc + col) * 2) : OOB;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((__vector_size__(16))) int, w), od,
                                                 off, 0, 2);
        }
        __builtin_amdgcn_wave_barrier();
      }
      if (c + 1 < nc) {
        // chunk c + 1 has landed once at most the memory operations issued
        // after its copies are outstanding
        if constexpr (SLOTS == 2) {
          wait_vm<OPS>();
        } else {
          if (c == 0) {
            if (ahead) wait_vm<J + OPS>();
            else wait_vm<OPS>();
          } else {
            if (ahead) wait_vm<OPS + J + OPS>();
            else wait_vm<OPS + OPS>();
          }
        }
        barrier();  // every wave's copies of chunk c + 1 are in LDS; slot of chunk c is free
      }
    }
  }
};

}  // namespace qa
