// Ping-pong bf16 GEMM for gfx950: a 256x256 output tile, 8 waves, BK 64,
// direct-to-LDS copies, and the two waves of every SIMD working in opposite
// phases.
//
// Waves 0-3 (group X, one per SIMD) and waves 4-7 (group Y, one per SIMD)
// each own a 128x64 block of the tile (group X the first 128 rows, group Y
// the last).  A K step is split into a memory phase (read every fragment of
// the step from LDS into registers, 24 fragments per wave, then issue this
// wave's copies) and a compute phase (32 back-to-back
// v_mfma_f32_32x32x16_bf16 from registers).  Group Y runs one phase behind
// group X and a workgroup barrier separates the phases, so while one wave of
// a SIMD issues its MFMAs the other issues its memory instructions.
//
// Phase t (between barriers t and t+1):
//   t = 2k     X reads step k, copies A(k+1);       Y multiplies step k-1
//   t = 2k+1   X multiplies step k, waits for A(k+1); Y reads step k,
//              copies B(k+2), waits for B(k+1)
// A lives in two LDS slots and B in three (160 KiB), so no copy overwrites a
// slot that a wave still reads, and every copy has about two phases to land.
// Every wave executes 2 nk + 1 barriers: X one before the loop and two per
// step, Y two before the loop, two per step but none after its last compute
// phase (it then writes its results while nothing else waits).
//
// Measured against GemmKernel's 256x256 tile (same box, rocprofv3 trace):
// 1-3% faster for the NN, NT and TT forms on 4096^3 and 8192-class shapes,
// equal to 1% slower for TN.  Both kernels run at the chip's power limit:
// schedules that stall less (fewer SQ_WAIT_ANY cycles) run at a higher clock
// (GRBM_GUI_ACTIVE per microsecond) for the same wall time, so the gain is
// small although the MFMA phases issue back to back.
//
// Results are bit-identical to GemmKernel's 256x256 tiles: the same LDS
// layout and fragment reads, the same MFMA per (row block, column block,
// 16-wide k step), and the same K order.
//
// Preconditions (checked by the host): bf16 operands with 16-byte aligned
// rows, K a positive multiple of 64, a plain or strided-batch product (no
// groups, split K, second K segment or SwiGLU).  Rows and columns beyond M
// and N need no masking: a copy descriptor spans exactly from the step's
// first element to the operand's last one, so nothing outside the operand is
// read, and values read past a row end only reach output rows or columns
// beyond M or N, which are never stored.
#pragma once
#include <type_traits>

#include "gemm_kernel.h"

namespace qa {

template <bool TA, bool TB>
struct PingPong {
  typedef GemmKernel<false, TA, TB, 256, 256, 2, 4, 64, 2, true> Base;
  typedef bf16_t T;
  static constexpr int NT = 512, BM = 256, BN = 256, BK = 64;
  static constexpr int TM = 128, TN = 64, FM = 4, FN = 2, S = BK / 16;
  static constexpr bool KA = !TA, KB = TB;
  static constexpr int TILE_BYTES = 256 * BK * 2;      // one operand's stage: 32 KiB
  static constexpr int STAGE_BYTES = 2 * TILE_BYTES;   // A then B
  static constexpr int LDS_BYTES = 5 * TILE_BYTES;  // A in two slots, B in three
  static_assert(LDS_BYTES >= 2 * STAGE_BYTES && LDS_BYTES >= Base::LDS_BYTES && LDS_BYTES <= 160 * 1024, "LDS");

  __device__ static __forceinline__ void barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
  // s_waitcnt lgkmcnt(0) with vmcnt / expcnt left at their maxima
  __device__ static __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

  // buffer_load_dwordx4 ... lds of 16 bytes per lane through descriptor d
  // (beyond its range: zeros) to LDS byte address m0 (lane l at m0 + 16 l).
  // Same contract as lds_load16, with the LDS address as a plain 32-bit
  // value (address 0 is a valid LDS address, not a null pointer).
  __device__ static __forceinline__ void copy16(u32x4 d, uint32_t m0, uint32_t voffset) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voffset), "s"(d)
                 : "memory", "m0");
  }

  // Lane part of the byte offset of copy instruction j of X wave w4 (the
  // row or k-row part that grows with j goes into the descriptor base).
  // K-major tile [256][64] (8 chunks per row): instruction j fills rows
  // 8 (4 j + w4) .. +7, lane l row 8 (4 j + w4) + l / 8, physical chunk l % 8,
  // i.e. logical chunk (l % 8) ^ swz_k(row), which depends on j only
  // through j % 2.
  __device__ static __forceinline__ uint32_t kmajor_lane(int64_t ld, int w4, int lane, int parity) {
    const int row = 8 * w4 + (lane >> 3);
    const int c = (lane & 7) ^ (((lane >> 3) ^ (4 * parity + w4)) & 7);
    return (uint32_t)(((int64_t)row * ld + c * 8) * 2);
  }
  // MN-major tile [64][256] (32 chunks per k-row): instruction j fills
  // k-rows 2 (4 j + w4) and +1, lane l k-row 2 (4 j + w4) + l / 32, physical
  // chunk l % 32 = logical chunk ^ swz_mn16(k-row), independent of j.
  __device__ static __forceinline__ uint32_t mnmajor_lane(int64_t ld, int w4, int lane) {
    const int krow = 2 * w4 + (lane >> 5);
    const int c = (lane & 31) ^ ((krow & 3) * 4);
    return (uint32_t)(((int64_t)krow * ld + c * 8) * 2);
  }

  // ---- fragment reads ------------------------------------------------------
  // The same LDS layout and lane assignment as GemmKernel::frag_k16 /
  // frag_mn16, with the per-lane part of every address computed once and the
  // rest (32-row block, 16-wide k step, second transpose read) an immediate
  // offset of the LDS instruction.
  //
  // K-major [256][64] slot, 8 chunks per row: lane l reads row
  // r = base + 32 b + l % 32 at logical chunk c = 2 s + l / 32, physical
  // chunk c ^ swz_k(r) with swz_k(r) = (r ^ (r >> 3)) & 7.  For base a
  // multiple of 32 that is t ^ 2 s ^ 4 (b & 1) with the lane's
  // t = l / 32 ^ (l % 8) ^ (l % 32) / 8, so four lane offsets serve every
  // block and step: off[x] = (base + l % 32) * 128 + 16 (t ^ 2 x), block b
  // and step s read off[s ^ 2 (b & 1)] + 4096 b.
  __device__ static __forceinline__ void kmajor_offsets(int base, int lane, uint32_t (&off)[4]) {
    const int rl = lane & 31, t = (lane >> 5) ^ (rl & 7) ^ (rl >> 3);
#pragma unroll
    for (int x = 0; x < 4; x++) off[x] = (uint32_t)((base + rl) * 128 + 16 * (t ^ (2 * x)));
  }
  // MN-major [64][256] slot, 32 chunks per k-row, read with
  // ds_read_b64_tr_b16: within a 16-lane group g = l / 16, lane i = l % 16
  // reads k-row k0 = 16 s + 8 (g / 2) + i / 4 (and k0 + 4) at column
  // cb = col + 16 (g & 1) + 4 (i % 4), chunk cb / 8 ^ 4 (i / 4) (swz_mn16 of
  // k0 and of k0 + 4).  For col = 32 (c0 + b) that is
  // 4 ((c0 + b) ^ i / 4) + 2 (g & 1) + (i % 4) / 2, so one lane offset per
  // 32-column block b: off[b] = k-row part + 16 chunk + 8 (i & 1), step s at
  // + 8192 s and the second read at + 2048.
  template <int NB>
  __device__ static __forceinline__ void mnmajor_offsets(int c0, int lane, uint32_t (&off)[NB]) {
    const int g = lane >> 4, i = lane & 15, q = i >> 2;
    const int cl = 2 * (g & 1) + ((i & 3) >> 1);
#pragma unroll
    for (int b = 0; b < NB; b++)
      off[b] = (uint32_t)(((g >> 1) * 8 + q) * 512 + 16 * (4 * ((c0 + b) ^ q) + cl) + 8 * (i & 1));
  }
  typedef __attribute__((address_space(3))) char lds_char;
  __device__ static __forceinline__ bf16x8 ld_k(uint32_t addr, int imm) {
    return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>(
        reinterpret_cast<const lds_char*>((uintptr_t)addr) + imm);
  }
  __device__ static __forceinline__ bf16x8 ld_mn(uint32_t addr, int imm) {
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    const lds_char* p = reinterpret_cast<const lds_char*>((uintptr_t)addr) + imm;
    i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
    i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 2048));
    i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, v);
  }

  __device__ static __forceinline__ void run(const GemmArgs& p, char* smem) {
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform32(tid >> 6);
    const int grp = wave >> 2, w4 = wave & 3;
    const int wm = grp, wn = w4;

    // ---- tile scheduling (as GemmKernel's plain products) -----------------
    const int tiles_n = (int)((p.N + BN - 1) / BN);
    const int tiles_m = p.tiles_m;
    const int total = (int)gridDim.x;
    const int tiles_per = tiles_m * tiles_n;
    const int pid = uniform32(xcd_remap((int)blockIdx.x, total));
    const int64_t bz = pid / tiles_per;
    const int t = pid % tiles_per;
    constexpr int GM = 4;
    const int group = t / (GM * tiles_n);
    const int first_m = group * GM;
    const int gsize = min(tiles_m - first_m, GM);
    const int tile_m = first_m + (t % (GM * tiles_n)) % gsize;
    const int tile_n = (t % (GM * tiles_n)) / gsize;

    const T* A = uniform_ptr(reinterpret_cast<const T*>(p.a) + bz * p.sa);
    const T* B = uniform_ptr(reinterpret_cast<const T*>(p.b) + bz * p.sb);
    char* outp = uniform_ptr(reinterpret_cast<char*>(p.out) + bz * p.sc * (p.out_bf16 ? 2 : 4));
    const int64_t M = p.M, N = p.N, K = p.K, lda = p.lda, ldb = p.ldb;
    const int64_t row0 = uniform64((int64_t)tile_m * BM), col0 = uniform64((int64_t)tile_n * BN);
    const int nk = (int)(K / BK);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

    // ---- copies (group X only) ----------------------------------------------
    // Operand origin and extent: A rows [row0, M) (K-major: A[m][k]; MN-major:
    // A[k][m]), B columns [col0, N) (K-major: B[n][k]; MN-major: B[k][n]).
    // Elements from the tile origin to the end of the operand's last chunk:
    //   K-major:  (ext - o0 - 1) * ld + K            (K is a multiple of 64)
    //   MN-major: (K - 1) * ld + round8(ext) - o0
    // An MN-major extent that is not a multiple of 8 only occurs for an
    // operand re-laid out with a zero-padded pitch (the host's rule), whose
    // last row still holds round8(ext) elements; ending the range at ext
    // would cut the last chunk of the matrix in two.
    const int64_t a_end = KA ? (M - row0 - 1) * lda + K : (K - 1) * lda + (M + 7) / 8 * 8 - row0;
    const int64_t b_end = KB ? (N - col0 - 1) * ldb + K : (K - 1) * ldb + (N + 7) / 8 * 8 - col0;
    // ---- copies ---------------------------------------------------------------
    // LDS: A in two slots, then B in three (5 x 32 KiB).  Group X copies A of
    // step k+1 in its memory phase of step k (phase 2k, into the slot of step
    // k-1, last read by Y in phase 2k-1) and waits for it at the end of phase
    // 2k+1; group Y copies B of step k+2 in its memory phase of step k (phase
    // 2k+1, into the slot of step k-1, last read by Y in phase 2k-1) and waits
    // for B of step k+1 at the end of that phase.  Every memory phase thus
    // carries half a step's copies, 8 one-KiB instructions per wave, issued
    // after the wave's fragment reads.  (Copies issued inside the compute
    // phase cost more MFMA time than they save: measured 20-50 cycles of MFMA
    // issue per copy.)
    const bool xa = grp == 0;                // this wave copies A (else B)
    const bool kc = xa ? KA : KB;            // its operand is K-major
    const int64_t ld = xa ? lda : ldb;
    uint32_t vo[2];                          // lane offsets of copy j: vo[j % 2]
    if (kc) {
      vo[0] = kmajor_lane(ld, w4, lane, 0);
      vo[1] = kmajor_lane(ld, w4, lane, 1);
    } else {
      vo[0] = vo[1] = mnmajor_lane(ld, w4, lane);
    }
    // copy instruction j of a step: K-major 32 rows further, MN-major 8 k-rows
    const uint32_t step_bytes = uniform32((uint32_t)((kc ? 32 : 8) * ld * 2));
    const T* tile = xa ? (KA ? A + row0 * lda : A + row0) : (KB ? B + col0 * ldb : B + col0);
    const int64_t end = xa ? a_end : b_end;  // elements from the tile origin to the operand's end
    const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_ptr_t)smem;
    auto a_slot = [&](int k) { return lds_base + (uint32_t)(k & 1) * TILE_BYTES; };
    auto b_slot = [&](int k) { return lds_base + (uint32_t)(2 + k % 3) * TILE_BYTES; };
    // this wave's copies of step k: descriptor base at the step's first
    // element, bytes from it to the operand's end (clamped to the
    // descriptor's 31-bit range; one instruction reaches at most 32 rows, far
    // below it, so the clamp never cuts a copy short), LDS destination
    auto copies = [&](int k) {
      const int64_t k0 = (int64_t)k * BK, kk = kc ? k0 : k0 * ld;
      const int64_t r64 = (end - kk) * 2;
      const uint64_t base = (uint64_t)(uintptr_t)tile + (uint64_t)kk * 2;
      const uint32_t range = uniform32(r64 <= 0 ? 0u : r64 > 0x7ffffff0 ? 0x7ffffff0u : (uint32_t)r64);
      const uint32_t dst = uniform32((xa ? a_slot(k) : b_slot(k)) + w4 * 1024);
      // one descriptor for the step's eight copies, instruction j's rows at
      // + j * step_bytes in the lane offset: lane bytes at or past `range`
      // read zeros exactly as with a descriptor based at the instruction's
      // own rows (range - j * step_bytes left), and the offsets stay below
      // 256 rows of the operand (< 2^31 bytes, the host's check)
      const u32x4 d = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base),
                       (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32) & 0xffffu),
                       (uint32_t)__builtin_amdgcn_readfirstlane(range), 0x00020000u};
#pragma unroll
      for (int j = 0; j < 8; j++) copy16(d, dst + j * 4096, vo[j & 1] + j * step_bytes);
    };

    // ---- fragment reads and products --------------------------------------------
    // per-lane fragment offsets inside a slot (A: 4 K-major offsets or one per
    // row block; B: 4 K-major offsets or one per column block)
    uint32_t oa[4], ob[4];
    if constexpr (KA) kmajor_offsets(wm * TM, lane, oa);
    else mnmajor_offsets<4>(wm * TM / 32, lane, oa);
    if constexpr (KB) kmajor_offsets(wn * TN, lane, ob);
    else mnmajor_offsets<2>(wn * TN / 32, lane, reinterpret_cast<uint32_t(&)[2]>(ob));
    bf16x8 fa[S][FM], fb[S][FN];
    auto memory_phase = [&](int k) {
      uint32_t pa[4], pb[4];
#pragma unroll
      for (int x = 0; x < 4; x++) pa[x] = a_slot(k) + oa[x];
#pragma unroll
      for (int x = 0; x < (KB ? 4 : 2); x++) pb[x] = b_slot(k) + ob[x];
#pragma unroll
      for (int st = 0; st < S; st++) {
#pragma unroll
        for (int i = 0; i < FM; i++) fa[st][i] = KA ? ld_k(pa[st ^ (2 * (i & 1))], 4096 * i) : ld_mn(pa[i], 8192 * st);
#pragma unroll
        for (int j = 0; j < FN; j++) fb[st][j] = KB ? ld_k(pb[st ^ (2 * (j & 1))], 4096 * j) : ld_mn(pb[j], 8192 * st);
      }
    };
    auto compute_phase = [&]() {
#pragma unroll
      for (int st = 0; st < S; st++)
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[st][i], fb[st][j], acc[i][j], 0, 0, 0);
    };

    // prologue: A of step 0 (group X), B of steps 0 and 1 (group Y)
    for (int k = 0; k < (xa ? 1 : nk > 1 ? 2 : 1); k++) copies(k);
    wait_vmcnt<0>();
    barrier();                // step 0 is in LDS
    if (grp == 1) barrier();  // group Y starts one phase later
    for (int kt = 0; kt < nk; kt++) {
      // memory phase: fragments of step kt, then this wave's copies
      memory_phase(kt);
      const int next = xa ? kt + 1 : kt + 2;  // the step this wave copies now
      const bool copying = next < nk;
      if (copying) copies(next);
      wait_lds();
      if (!xa) {
        // B of step kt+1 is in LDS before the next barrier (the 8 copies
        // just issued may still be in flight)
        if (copying) wait_vmcnt<8>();
        else wait_vmcnt<0>();
      }
      barrier();
      compute_phase();
      if (xa) {
        wait_vmcnt<0>();  // A of step kt+1 is in LDS before the next barrier
        barrier();
      } else if (kt + 1 < nk) {
        barrier();
      }
    }

    // ---- epilogue (GemmKernel's): every ring read ended before the last
    // barrier, so the per-wave staging areas are free -------------------------
    typename Base::Out o;
    o.ptr = outp;
    o.ldc = p.ldc;
    o.M = M;
    o.N = N;
    o.row0 = row0 + wm * TM;
    o.col0 = col0 + wn * TN;
    o.bf16 = p.out_bf16;
    o.accumulate = p.accumulate;
    o.vec = p.vec_c;
    o.alpha = p.alpha;
    float* stage = reinterpret_cast<float*>(smem) + wave * 32 * Base::EP;
    const bool fast = o.vec >= (o.bf16 ? 2 : 1) && o.row0 + TM <= o.M && o.col0 + TN <= o.N;
#pragma unroll
    for (int i = 0; i < FM; i++) Base::template store_slab<FN>(acc[i], stage, o, o.row0 + i * 32, lane, fast);
  }
};

}  // namespace qa
