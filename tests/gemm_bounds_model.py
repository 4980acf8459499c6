"""Host model of the GEMM kernels' memory addressing (CPU only).

Every operand load of the MFMA GEMM kernels is a 16-byte buffer load whose
address is a descriptor base plus a per-lane byte offset; a load that the
kernel decides is outside the matrix gets the offset 0x80000000, beyond the
descriptor's range, and reads zeros.  Whether the remaining loads stay inside
the operand's allocation rests on host-side invariants (16-byte aligned K-major
rows, zero-padded re-layouts, split-K chunks of a multiple of 64, ...), not on
the descriptor range, which starts at the tile's first row and may extend past
the allocation.  This module restates, with numpy, the offsets the kernels
compute -- per tile, K step, copy instruction and lane -- so that tests can
check over randomised shapes that every issued load and every store lies
inside its allocation.

Restated from qutai_amd/csrc/gemm_kernel.h (tile scheduling and operand
bases 342-404, descriptor bases 418-425 and 466-471, DMA lane offsets
430-465, register-staging offsets 523-545, epilogue 590-660 and 711-770) and
qutai_amd/csrc/gemm_short.h (copies 91-101, output offsets 104-112 and
176-186); the host's operand re-layout rule (plan_operand), split-K chunking
(choose_split), grouped grid and the pair form's K join from
qutai_amd/csrc/gemm.hip.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

OOB = 0x80000000
RANGE_CAP = 0x7FFFFFF0


@dataclass(frozen=True)
class Config:
    """One kernel configuration: GemmKernel<F32, TA, TB, BM, BN, WM, WN, BK, STAGES, DMA, SWIGLU>."""
    name: str
    bm: int
    bn: int
    wm: int
    wn: int
    bk: int
    stages: int
    dma: bool = True
    swiglu: bool = False


def tile_configs(f32: bool) -> list[Config]:
    """The tile table of launch_tile (gemm.hip): K per stage 64/32 (bf16/fp32)
    for the two- and three-stage rings, 32/16 for the four-stage ones; T and U
    are 256x256 for fp32."""
    kb, kr = (16, 32) if f32 else (32, 64)
    table = [Config("L8D2", 256, 256, 2, 4, kr, 2), Config("L8R", 256, 256, 2, 4, kr, 2, dma=False),
             Config("L4D2", 256, 256, 2, 2, kr, 2), Config("S", 128, 128, 2, 2, kb, 4),
             Config("S2", 128, 128, 2, 2, kb, 2), Config("N", 256, 64, 4, 1, kr, 2),
             Config("W", 64, 256, 1, 4, kb, 4), Config("H", 256, 128, 4, 2, kr, 3)]
    if f32:
        table += [Config("T", 256, 256, 2, 4, kr, 2), Config("U", 256, 256, 2, 4, kr, 2)]
    else:
        table += [Config("T", 192, 256, 2, 4, kr, 2), Config("U", 256, 192, 4, 2, kr, 2)]
    return table


SWIGLU = Config("SWIGLU", 256, 256, 2, 4, 64, 2, swiglu=True)


# ---- LDS chunk maps (OperandTile::coords) -------------------------------------------

def _swz_k(ck: int, r: np.ndarray) -> np.ndarray:
    return (r ^ (r >> 3)) & 7 if ck == 8 else ((r >> 1) ^ (r >> 3)) & 3


def _swz_mn(f32: bool, cr: int, k: np.ndarray) -> np.ndarray:
    if f32:
        return ((k >> 3) & 1) * 8
    return (k & 3) * 4 if cr % 16 == 0 else ((k >> 1) & 1) * 4


def chunk_coords(f32: bool, kmajor: bool, rows: int, bk: int, q: np.ndarray):
    """(outer, logical chunk) of physical chunk q of a [rows][bk] (K-major) or
    [bk][rows] (MN-major) operand stage."""
    e = 4 if f32 else 8
    if kmajor:
        ck = bk // e
        outer = q // ck
        return outer, (q % ck) ^ _swz_k(ck, outer)
    cr = rows // e
    outer = q // cr
    return outer, (q % cr) ^ _swz_mn(f32, cr, outer)


@dataclass
class Operand:
    """An operand as the kernel sees it: element strides and the allocation
    (in elements) that its loads must stay inside."""
    ld: int
    batch_stride: int
    alloc: int


class Violation(AssertionError):
    pass


def _check(what: str, lo: np.ndarray, hi: np.ndarray, alloc_bytes: int):
    """Byte ranges [lo, hi) must lie in [0, alloc_bytes)."""
    if lo.size == 0:
        return
    if lo.min() < 0 or hi.max() > alloc_bytes:
        bad = np.flatnonzero((lo < 0) | (hi > alloc_bytes))[0]
        raise Violation(f"{what}: access [{lo.flat[bad]}, {hi.flat[bad]}) outside [0, {alloc_bytes})")


def operand_loads(cfg: Config, f32: bool, kmajor: bool, rows_tile: int, base_elem: int, row0: int, rows: int,
                  k_len: int, ld: int, alloc: int, what: str, gather: np.ndarray | None = None,
                  swiglu_up: bool = False, index_check: bool = True):
    """Every load of one operand over one tile's K loop: base_elem is the
    operand pointer after the mode's adjustments (in elements), row0 the
    tile's first row (A) / column (B), rows the operand's valid extent (M or
    N), k_len the K range.  gather (grouped A, K-major): row i of the tile's
    group is row gather[row0 + i] of the operand, the descriptor spans the
    whole allocation, the byte offset is a 32-bit value, and an index
    outside the operand's rows gets the out-of-range offset (index_check;
    without it -- a planted mistake -- such an index is issued with its
    wrapped offset, and one that wraps onto a real row is reported)."""
    e, es = (4, 4) if f32 else (8, 2)
    nt = 64 * cfg.wm * cfg.wn
    chunks = rows_tile * cfg.bk // e
    if cfg.dma:
        q = np.arange(chunks)  # physical chunk (j * NW + wave) * 64 + lane
        outer, c = chunk_coords(f32, kmajor, rows_tile, cfg.bk, q)
    else:  # register staging: thread idx = tid + i * NT walks the chunks row by row
        idx = np.arange(chunks)
        per = cfg.bk // e if kmajor else rows_tile // e
        outer, c = idx // per, idx % per
    if cfg.swiglu and what.startswith("B"):
        # tile row `outer` is row (outer / 64) * 32 + outer % 32 of the gate
        # or up weight (the same offsets for both, each its own descriptor)
        outer = ((outer >> 6) << 5) + (outer & 31)
    kidx = c * e if kmajor else outer
    valid = (row0 + outer < rows) if kmajor else (row0 + c * e < rows)
    if gather is not None:
        src = np.where(valid, gather[np.minimum(row0 + outer, gather.size - 1)], outer)
        outside = valid & ((src < 0) | (src >= alloc // ld))
        off = ((src * ld + c * e) * es) & 0xFFFFFFFF  # the kernel's uint32 byte offset
        if index_check:
            valid = valid & ~outside
        elif np.any(outside & (off + 16 <= min(alloc * es, RANGE_CAP))):
            raise Violation(f"{what}: a gathered index outside the operand reads a real row")
    else:
        off = (outer * ld + c * e) * es
    nk = (k_len + cfg.bk - 1) // cfg.bk
    for kt in range(nk):
        k0 = kt * cfg.bk
        krem = k_len - k0
        if gather is not None:
            tile_elem = base_elem + k0
            span = alloc * es
        else:
            tile_elem = base_elem + (row0 * ld + k0 if kmajor else k0 * ld + row0)
            span = (rows_tile * ld if kmajor else cfg.bk * ld) * es
        rng = min(span, RANGE_CAP)
        issued = valid & (kidx < krem)
        offs = np.where(issued, off, OOB)
        hit = offs + 16 <= rng  # the load reads memory (else zeros)
        if np.any(issued & ~hit):
            raise Violation(f"{what}: an in-matrix chunk falls outside the descriptor range")
        lo = tile_elem * es + offs[hit]
        _check(f"{what} load", lo, lo + 16, alloc * es)


def output_stores(cfg: Config, f32_out: bool, out_elem: int, row0: int, col0: int, m: int, n: int, ldc: int,
                  alloc: int, vec: int, what: str = "C"):
    """Element ranges the epilogue writes for one tile (store_slab / write4):
    the straight-line path for a whole in-range wave tile with aligned rows,
    else per 4 columns with row < M and col < N checks."""
    es = 4 if f32_out else 2
    tm = cfg.bm // cfg.wm
    bno = cfg.bn // 2 if cfg.swiglu else cfg.bn
    tw = bno // cfg.wn
    for wm in range(cfg.wm):
        for wn in range(cfg.wn):
            r0, c0 = row0 + wm * tm, col0 + wn * tw
            fast = vec >= (1 if f32_out else 2) and r0 + tm <= m and c0 + tw <= n
            if fast:
                rows = np.arange(r0, r0 + tm)
                lo = (out_elem + rows * ldc + c0) * es
                _check(f"{what} store (fast)", lo, lo + tw * es, alloc * es)
            else:
                rows = np.arange(r0, min(r0 + tm, m))
                if rows.size == 0 or c0 >= n:
                    continue
                last = min(c0 + tw, n)
                lo = (out_elem + rows * ldc + c0) * es
                _check(f"{what} store", lo, lo + (last - c0) * es, alloc * es)


def plan_operand(inner: int, outer: int, batch: int, stride: int, f32_compute: bool, aligned_base: bool = True):
    """plan_operand (gemm.hip): rows of `inner` elements are used in place when
    16-byte aligned (inner a multiple of E, batch stride too), else re-laid out
    into a zero-padded pitch.  Returns (ld, batch stride, allocation) as the
    kernel sees the operand."""
    e = 4 if f32_compute else 8
    alloc = (batch - 1) * stride + outer * inner if stride else outer * inner
    if aligned_base and inner % e == 0 and (batch <= 1 or stride % e == 0):
        return Operand(inner, stride, alloc)
    pitch = (inner + e - 1) // e * e
    batches = 1 if stride == 0 or batch <= 1 else batch
    return Operand(pitch, 0 if stride == 0 else outer * pitch, batches * outer * pitch)


def split_chunk(inner: int, splits: int) -> tuple[int, int]:
    """choose_split's chunking: chunks of a multiple of 64 elements."""
    c = ((inner + splits - 1) // splits + 63) // 64 * 64
    return (inner + c - 1) // c, c


def plain_gemm(cfg: Config, f32: bool, m: int, k: int, n: int, batch: int, ta: bool, tb: bool,
               broadcast_a: bool = False, broadcast_b: bool = False, splits: int = 1, out_f32: bool = True):
    """All loads and stores of one qutai_amd_gemm call on tile `cfg`
    (batched, broadcast operands, optional split-K into fp32 partials)."""
    pa = plan_operand(m if ta else k, k if ta else m, batch, 0 if broadcast_a else m * k, f32)
    pb = plan_operand(k if tb else n, n if tb else k, batch, 0 if broadcast_b else k * n, f32)
    ka, kb = not ta, tb
    chunk = k
    if splits > 1:
        splits, chunk = split_chunk(k, splits)
        out_f32 = True
    tiles_m, tiles_n = (m + cfg.bm - 1) // cfg.bm, (n + cfg.bn - 1) // cfg.bn
    out_alloc = splits * batch * m * n
    vec = 2 if n % 8 == 0 else 1 if n % 4 == 0 else 0
    for z in range(batch * splits):
        prod, s = divmod(z, splits)
        k_lo = s * chunk
        k_len = min(k, k_lo + chunk) - k_lo
        a_base = prod * pa.batch_stride + k_lo * (1 if ka else pa.ld)
        b_base = prod * pb.batch_stride + k_lo * (1 if kb else pb.ld)
        for tm in range(tiles_m):
            for tn in range(tiles_n):
                operand_loads(cfg, f32, ka, cfg.bm, a_base, tm * cfg.bm, m, k_len, pa.ld, pa.alloc, "A")
                operand_loads(cfg, f32, kb, cfg.bn, b_base, tn * cfg.bn, n, k_len, pb.ld, pb.alloc, "B")
                output_stores(cfg, out_f32, z * m * n, tm * cfg.bm, tn * cfg.bn, m, n, n, out_alloc, vec)



def window_gemm(cfg: Config, f32: bool, m: int, k: int, n: int, c0: int, width: int, ta: bool, tb: bool,
                splits: int = 1, out_f32: bool = True):
    """One column window [c0, c0 + width) of a plain product (the column
    remainder's two launches, column_split / plan_windows): B from its c0-th
    column (row when K-major), out from column c0 at the full pitch n; with
    split K the fp32 partials are [m][width] each."""
    pa = plan_operand(m if ta else k, k if ta else m, 1, m * k, f32)
    pb = plan_operand(k if tb else n, n if tb else k, 1, k * n, f32)
    ka, kb = not ta, tb
    chunk = k
    if splits > 1:
        splits, chunk = split_chunk(k, splits)
    b_shift = c0 * (pb.ld if kb else 1)
    tiles_m, tiles_n = (m + cfg.bm - 1) // cfg.bm, (width + cfg.bn - 1) // cfg.bn
    for s in range(splits):
        k_lo = s * chunk
        k_len = min(k, k_lo + chunk) - k_lo
        a_base = k_lo * (1 if ka else pa.ld)
        b_base = b_shift + k_lo * (1 if kb else pb.ld)
        for tm in range(tiles_m):
            for tn in range(tiles_n):
                operand_loads(cfg, f32, ka, cfg.bm, a_base, tm * cfg.bm, m, k_len, pa.ld, pa.alloc, "A")
                operand_loads(cfg, f32, kb, cfg.bn, b_base, tn * cfg.bn, width, k_len, pb.ld, pb.alloc, "B")
                if splits > 1:
                    vec = 2 if width % 8 == 0 else 1 if width % 4 == 0 else 0
                    output_stores(cfg, True, s * m * width, tm * cfg.bm, tn * cfg.bn, m, width, width,
                                  splits * m * width, vec, "partial")
                else:
                    vec = 2 if n % 8 == 0 else 1 if n % 4 == 0 else 0
                    output_stores(cfg, out_f32, c0, tm * cfg.bm, tn * cfg.bn, m, width, n, m * n, vec)


def remainder_rows(f32: bool, m: int, k: int, n: int, c0: int, width: int, tb: bool, b_source: bool = False,
                   b_f32: bool | None = None):
    """remainder_columns / prepare_remainder (gemm.hip): the last `width` <= 8
    columns of a plain product with a K-major A.  Each workgroup stages B's
    elements (k, c0 + j), k < K, j < width, KC values of k at a time
    into an LDS block [8][KC] (KC = 1024); B is the planned operand, or with b_source the
    caller's own B (source pitch and dtype b_f32) that the fused re-layout
    launch reads.  Each wave row m < M reads A's row in 16-byte chunks
    c * E < K (KC / E chunks per staged block) and the block's matching
    values; out's (m, c0 + j) at pitch n."""
    e, es = (4, 4) if f32 else (8, 2)
    kc = 1024
    pa = plan_operand(k, m, 1, m * k, f32)
    if b_source:
        b_f32 = f32 if b_f32 is None else b_f32
        ld, alloc, bes = (k if tb else n), k * n, (4 if b_f32 else 2)
    else:
        pb = plan_operand(k if tb else n, n if tb else k, 1, k * n, f32)
        ld, alloc, bes = pb.ld, pb.alloc, es
    kk = np.arange(k)[:, None]
    j = np.arange(width)[None, :]
    at = ((c0 + j) * ld + kk) if tb else (kk * ld + c0 + j)
    _check("remainder B load", at.ravel() * bes, at.ravel() * bes + bes, alloc * bes)
    for k0 in range(0, k, kc):
        chunks = np.arange((min(k - k0, kc) + e - 1) // e)
        if chunks.size * e > kc:
            raise Violation("remainder: a chunk past the staged LDS block")
        lo = ((np.arange(m)[:, None] * pa.ld + k0 + chunks[None, :] * e) * es).ravel()
        _check("remainder A load", lo, lo + 16, pa.alloc * es)
    at = (np.arange(m)[:, None] * n + c0 + j).ravel()
    _check("remainder store", at * 4, at * 4 + 4, m * n * 4)


def grouped_gemm(cfg: Config, f32: bool, counts: list[int], inner: int, cols: int, transpose_right: bool,
                 gather: np.ndarray | None = None, source_rows: int = 0, index_check: bool = True):
    """qutai_amd_gemm_grouped (and the SwiGLU form with cfg = SWIGLU): group g
    owns rows [offsets[g], offsets[g+1]) of A (or, with gather, the rows
    gather[offsets[g]:...] of a source_rows-row A) and of out; its B is
    b + g * expert_stride."""
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    capacity = int(offsets[-1])
    groups = len(counts)
    es_in = 4 if f32 else 2
    ldb = inner if transpose_right else cols
    expert_stride = cols * inner
    a_alloc = (source_rows if gather is not None else capacity) * inner
    b_alloc = groups * expert_stride
    bno = cfg.bn // 2 if cfg.swiglu else cfg.bn
    tiles_n = (cols + bno - 1) // bno
    vec = 2 if cols % 8 == 0 else 1 if cols % 4 == 0 else 0
    # the entry point's own checks (QA_EINVAL otherwise): 16-byte rows
    e = 4 if f32 else 8
    if inner % e or ldb % e or (inner * 256 * es_in) >= 2 ** 31 or (ldb * 256 * es_in) >= 2 ** 31:
        raise ValueError("rejected by qutai_amd_gemm_grouped")
    for g in range(groups):
        lo, hi = int(offsets[g]), int(offsets[g + 1])
        rows = hi - lo
        for tm in range((rows + cfg.bm - 1) // cfg.bm):
            row0 = tm * cfg.bm
            if gather is not None:
                operand_loads(cfg, f32, True, cfg.bm, 0, row0, rows, inner, inner, a_alloc, "A",
                              gather=gather[lo:hi], index_check=index_check)
            else:
                operand_loads(cfg, f32, True, cfg.bm, lo * inner, row0, rows, inner, inner, a_alloc, "A")
            for tn in range(tiles_n):
                col0 = tn * bno
                if cfg.swiglu:  # gate and up weights: one 32-row block each in turn
                    for up in (False, True):
                        operand_loads(cfg, f32, True, cfg.bn, g * expert_stride, col0, cols, inner, ldb, b_alloc,
                                      "B" + ("up" if up else "gate"), swiglu_up=up)
                else:
                    operand_loads(cfg, f32, transpose_right, cfg.bn, g * expert_stride, col0, cols, inner, ldb,
                                  b_alloc, "B")
                output_stores(cfg, False, lo * cols, row0, col0, rows, cols, cols, capacity * cols, vec)


def grouped_pair_gemm(cfg: Config, f32: bool, counts: list[int], inner: int, cols: int, transpose_right: bool):
    """qutai_amd_gemm_grouped_pair: one grouped product over K = 2 inner whose
    steps below inner read (a, b) and the rest (a_tail, b_tail) at k - inner,
    two allocations per side of the grouped shapes.  inner is a multiple of 64
    (the entry point's check), so every step of the first half is whole and
    each half's loads are those of a grouped product over K = inner."""
    if inner % 64 or inner == 0:
        raise ValueError("rejected by qutai_amd_gemm_grouped_pair")
    for _ in ("head", "tail"):
        grouped_gemm(cfg, f32, counts, inner, cols, transpose_right)


def gathered_k_loads(cfg: Config, f32: bool, col0: int, cols: int, k_lo: int, k_len: int, gather: np.ndarray,
                     source_rows: int, index_check: bool = True):
    """Every load of an MN-major B whose K rows are gathered (GATHER_B): the
    chunk of k row `outer` in the step at k0 reads row gather[k_lo + k0 +
    outer] of the [source_rows][cols] matrix -- the index is read only for
    k0 + outer < k_len and a column inside N, so the table is never read past
    the group -- through a descriptor based at column col0 that spans the
    rest of the matrix, with a 32-bit byte offset; an index outside the rows
    gets the out-of-range offset (without index_check -- a planted mistake --
    it is issued with its wrapped offset, and one that lands on a real row is
    reported)."""
    e, es = (4, 4) if f32 else (8, 2)
    if cfg.stages != 2 or not cfg.dma:
        raise ValueError("gathered K rows run on the two-stage direct-to-LDS tiles only")
    alloc = source_rows * cols
    q = np.arange(cfg.bn * cfg.bk // e)
    outer, c = chunk_coords(f32, False, cfg.bn, cfg.bk, q)
    valid = col0 + c * e < cols
    span = min(alloc * es - col0 * es, RANGE_CAP)
    for kt in range((k_len + cfg.bk - 1) // cfg.bk):
        k = kt * cfg.bk + outer
        read = valid & (k < k_len)
        at = k_lo + k[read]
        if at.size and (at.min() < 0 or at.max() >= gather.size):
            raise Violation("B: an index read outside the route order")
        src = np.full(q.size, -1, dtype=np.int64)
        src[read] = gather[at]
        inside = read & (src >= 0) & (src < source_rows)
        wrapped = ((src * cols) * es + c * e * es) & 0xFFFFFFFF
        issued = inside if index_check else read
        offs = np.where(issued, wrapped, OOB)
        hit = offs + 16 <= span
        if np.any(inside & ~hit):
            raise Violation("B (gathered): an in-matrix chunk falls outside the descriptor range")
        if not index_check and np.any(read & ~inside & hit):
            raise Violation("B (gathered): an index outside the source reads a real row")
        lo = col0 * es + offs[hit]
        _check("B (gathered) load", lo, lo + 16, alloc * es)


def grouped_k_gemm(cfg: Config, f32: bool, counts: list[int], rows: int, cols: int,
                   gather: np.ndarray | None = None, source_rows: int = 0, index_check: bool = True):
    """qutai_amd_gemm_grouped_k: out[g] = A_g^T B_g over the K rows
    [offsets[g], offsets[g+1]) of a [capacity][rows] and b [capacity][cols]
    (A and B MN-major, ta = 1, tb = 0); with gather, K row k of B is row
    gather[k] of a [source_rows][cols] token matrix (gathered_k_loads)."""
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    capacity = int(offsets[-1])
    pa = plan_operand(rows, capacity, 1, 0, f32)
    pb = plan_operand(cols, capacity, 1, 0, f32)
    tiles_m, tiles_n = (rows + cfg.bm - 1) // cfg.bm, (cols + cfg.bn - 1) // cfg.bn
    vec = 2 if cols % 8 == 0 else 1 if cols % 4 == 0 else 0
    for g in range(len(counts)):
        k_lo, k_hi = int(offsets[g]), int(offsets[g + 1])
        for tm in range(tiles_m):
            for tn in range(tiles_n):
                operand_loads(cfg, f32, False, cfg.bm, k_lo * pa.ld, tm * cfg.bm, rows, k_hi - k_lo, pa.ld,
                              pa.alloc, "A")
                if gather is not None:
                    gathered_k_loads(cfg, f32, tn * cfg.bn, cols, k_lo, k_hi - k_lo, gather, source_rows,
                                     index_check)
                else:
                    operand_loads(cfg, f32, False, cfg.bn, k_lo * pb.ld, tn * cfg.bn, cols, k_hi - k_lo, pb.ld,
                                  pb.alloc, "B")
                output_stores(cfg, True, g * rows * cols, tm * cfg.bm, tn * cfg.bn, rows, cols, cols,
                              len(counts) * rows * cols, vec)


def short_strip(m: int, k: int, n: int, batch: int, strip: int):
    """The short-K strip kernel (gemm_short.h): A block [128][64] and B chunks
    through descriptors starting at the block's / chunk's first row with a
    128-row range; output 16-byte stores at row offsets inside the tile's
    existing rows and columns below N (N a multiple of 16)."""
    assert k <= 64 and n % 16 == 0
    pa = plan_operand(k, m, batch, m * k, False)
    pb = plan_operand(k, n, batch, n * k, False)
    cfg = Config("R", 128, 128, 2, 2, 64, 2)
    tiles_m, chunks = (m + 127) // 128, (n + 127) // 128
    # strip s sweeps chunks s, s + strips, ... (strips = ceil(chunks / strip)):
    # every chunk belongs to exactly one strip
    strips = (chunks + strip - 1) // strip
    covered = sorted(s + c * strips for s in range(strips) for c in range((chunks - s + strips - 1) // strips))
    assert covered == list(range(chunks))
    lane = np.arange(64)
    for z in range(batch):
        for tm in range(tiles_m):
            row0 = tm * 128
            # copy(): offsets (row * ld + chunk * 8) * 2 from A + row0 * lda
            operand_loads(cfg, False, True, 128, z * pa.batch_stride, row0, m, k, pa.ld, pa.alloc, "A")
            rows_here = min(128, m - row0)
            orange = min(rows_here * n * 2, RANGE_CAP)
            obase = (z * m * n + row0 * n) * 2
            for c in range(chunks):
                n0 = c * 128
                operand_loads(cfg, False, True, 128, z * pb.batch_stride, n0, n, k, pb.ld, pb.alloc, "B")
                for wm in range(2):
                    for wn in range(2):
                        for fm in range(2):
                            for it in range(4):
                                idx = it * 64 + lane
                                r, q = idx >> 3, idx & 7
                                col = n0 + wn * 64 + 8 * q
                                off = np.where(col < n, ((wm * 64 + fm * 32 + r) * n + col) * 2, OOB)
                                hit = off + 16 <= orange
                                lo = obase + off[hit]
                                _check("C store (strip)", lo, lo + 16, batch * m * n * 2)


# ---- ping-pong kernel (gemm_pingpong.h) ------------------------------------------------

PINGPONG = Config("P", 256, 256, 2, 4, 64, 2)


def _pingpong_lane(kmajor: bool, ld: int, w4: int, parity: int) -> np.ndarray:
    """PingPong::kmajor_lane / mnmajor_lane: byte offset of each lane of copy
    instruction j (parity j % 2) of wave w4 from the instruction's base."""
    lane = np.arange(64)
    if kmajor:
        row = 8 * w4 + (lane >> 3)
        c = (lane & 7) ^ (((lane >> 3) ^ (4 * parity + w4)) & 7)
    else:
        row = 2 * w4 + (lane >> 5)
        c = (lane & 31) ^ ((row & 3) * 4)
    return (row * ld + c * 8) * 2


def pingpong_operand(kmajor: bool, base_elem: int, o0: int, ext: int, k: int, ld: int, alloc: int, what: str,
                     range_rule: str = "end"):
    """Every copy of one operand over one tile's K loop in the ping-pong
    kernel: instruction j of wave w4 at step kt has descriptor base
    tile + kk + j * step (elements; step = 32 rows K-major, 8 k-rows
    MN-major) and range = bytes from the step's first element to the
    end of the operand's last chunk (range_rule "end", the kernel's: K-major
    rows end at K, a multiple of 64; MN-major rows at the extent rounded up to
    8, which the host's zero-padded re-layout guarantees), minus j * step,
    clamped to [0, RANGE_CAP].  Checks (1) every lane that reads memory
    reads inside the allocation, (2) every chunk of the matrix (row < ext,
    k < K) is read, not zeroed, and lands at the LDS position whose
    OperandTile coordinates are its own, and (3) the 32 instructions of a
    step fill each 16-byte chunk of the 32 KiB slot exactly once.
    range_rule "tile" (a planted mistake for the tests) spans the tile's
    256 rows instead of ending at the operand; "exact" ends MN-major rows at
    the extent itself, which cuts the last chunk of a ragged extent."""
    es = 2
    if k % 64 or k <= 0:
        raise ValueError("the ping-pong kernel needs K a positive multiple of 64")
    end = (ext - o0 - 1) * ld + k if kmajor else (k - 1) * ld + (ext + 7) // 8 * 8 - o0
    step_elems = 32 * ld if kmajor else 8 * ld
    tile = base_elem + (o0 * ld if kmajor else o0)
    lane = np.arange(64)
    for kt in range(k // 64):
        k0 = kt * 64
        kk = k0 if kmajor else k0 * ld
        if range_rule == "end":
            r0 = min(max((end - kk) * es, 0), RANGE_CAP)
        elif range_rule == "exact":
            r0 = min(max(((ext - o0 - 1) * ld + k if kmajor else (k - 1) * ld + ext - o0) - kk, 0) * es, RANGE_CAP)
        else:
            r0 = min((256 * ld if kmajor else 64 * ld) * es, RANGE_CAP)
        filled = np.zeros(256 * 64 // 8, dtype=np.int64)
        for w4 in range(4):
            for j in range(8):
                off = _pingpong_lane(kmajor, ld, w4, j & 1)
                rng = max(r0 - j * step_elems * es, 0)
                hit = off + 16 <= rng
                lo = (tile + kk + j * step_elems) * es + off[hit]
                _check(f"{what} copy", lo, lo + 16, alloc * es)
                # the element each lane fetches and where it lands in LDS
                q = (4 * j + w4) * 64 + lane
                outer, c = chunk_coords(False, kmajor, 256, 64, q)
                filled[q] += 1
                if kmajor:
                    src_outer, src_c = 32 * j + 8 * w4 + (lane >> 3), (off // es - (8 * w4 + (lane >> 3)) * ld) // 8
                else:
                    src_outer, src_c = 8 * j + 2 * w4 + (lane >> 5), (off // es - (2 * w4 + (lane >> 5)) * ld) // 8
                if not (np.array_equal(src_outer, outer) and np.array_equal(src_c, c)):
                    raise Violation(f"{what}: copy lands at the wrong LDS chunk")
                row_ok = (o0 + outer < ext) if kmajor else (o0 + c * 8 < ext)
                if np.any(row_ok & ~hit):
                    raise Violation(f"{what}: a chunk of the matrix falls outside the copy descriptor")
        if not np.all(filled == 1):
            raise Violation(f"{what}: LDS slot not filled exactly once")


def pingpong_gemm(m: int, k: int, n: int, batch: int, ta: bool, tb: bool, broadcast_a: bool = False,
                  broadcast_b: bool = False, range_rule: str = "end", out_f32: bool = False):
    """All copies and stores of one qutai_amd_gemm call on the ping-pong
    kernel (bf16, K a multiple of 64, batched or broadcast operands)."""
    pa = plan_operand(m if ta else k, k if ta else m, batch, 0 if broadcast_a else m * k, False)
    pb = plan_operand(k if tb else n, n if tb else k, batch, 0 if broadcast_b else k * n, False)
    tiles_m, tiles_n = (m + 255) // 256, (n + 255) // 256
    vec = 2 if n % 8 == 0 else 1 if n % 4 == 0 else 0
    for z in range(batch):
        for tm in range(tiles_m):
            for tn in range(tiles_n):
                pingpong_operand(not ta, z * pa.batch_stride, tm * 256, m, k, pa.ld, pa.alloc, "A", range_rule)
                pingpong_operand(tb, z * pb.batch_stride, tn * 256, n, k, pb.ld, pb.alloc, "B", range_rule)
                output_stores(PINGPONG, out_f32, z * m * n, tm * 256, tn * 256, m, n, n, batch * m * n, vec)
