"""CPU bounds model of the GEMM kernels' addressing (tests/gemm_bounds_model.py):
over randomised shapes -- ragged sizes, K not a multiple of the K step or of
the 16-byte chunk, odd pitches that force the host's re-layout, broadcast
batches, split-K chunks, empty and single-row experts, gathered rows -- every
load the kernels issue and every store they make lies inside its operand's
allocation, and every chunk inside the matrix is inside its descriptor's
range, for every tile configuration.  The model is checked first against the
fault class it exists for: a K-major operand whose rows are not 16-byte
aligned, or a K chunk that is not a multiple of 8, makes a 16-byte load run
past the row end -- in the last tile past the allocation -- and the model
must report it."""
import numpy as np
import pytest

from tests import gemm_bounds_model as gm

SEED = 20261202


def _shapes(rng, count, low=1, high=700):
    return [tuple(int(v) for v in rng.integers(low, high, size=3)) for _ in range(count)]


def test_model_reports_the_split_k_fault_class():
    """A planted mistake: K-major rows of 100 bf16 (200 bytes, not 16-byte
    aligned) used in place, and a K range of 100 that is not a multiple of
    8 -- the last chunk of the last row reads past the allocation."""
    cfg = gm.tile_configs(False)[0]
    m, k = 256, 100
    with pytest.raises(gm.Violation):
        gm.operand_loads(cfg, False, True, cfg.bm, 0, 0, m, k, k, m * k, "A")
    # the host's re-layout (pitch 104, zero padding) removes it
    op = gm.plan_operand(k, m, 1, 0, False)
    assert op.ld == 104
    gm.operand_loads(cfg, False, True, cfg.bm, 0, 0, m, k, op.ld, op.alloc, "A")


def test_model_reports_a_gather_index_past_the_source():
    """A route order entry outside the token rows reads zeros: equal to the
    row count, negative, or so large that its 32-bit byte offset wraps onto
    row 1 (2^32 / 128 + 1 rows of 64 bf16).  The planted mistake -- the
    kernel without its index check -- reads that real row, and the model
    reports it."""
    counts = [3, 0, 5]
    order = np.array([0, 1, 2, 3, 4, 5, 6, 7])
    cfg = gm.tile_configs(False)[0]
    gm.grouped_gemm(cfg, False, counts, 64, 32, True, gather=order, source_rows=8)
    for bad in (8, -1, (1 << 32) // 128 + 1):
        order[5] = bad
        gm.grouped_gemm(cfg, False, counts, 64, 32, True, gather=order, source_rows=8)
    with pytest.raises(gm.Violation):
        gm.grouped_gemm(cfg, False, counts, 64, 32, True, gather=order, source_rows=8, index_check=False)


@pytest.mark.parametrize("f32", [False, True], ids=["bf16", "fp32"])
def test_plain_and_batched_products_stay_in_bounds(f32):
    rng = np.random.default_rng(SEED + f32)
    shapes = _shapes(rng, 3) + [(257, 65, 129), (1, 1, 1), (300, 8, 31)]
    for cfg in gm.tile_configs(f32):
        for m, k, n in shapes:
            for ta in (False, True):
                for tb in (False, True):
                    gm.plain_gemm(cfg, f32, m, k, n, 1, ta, tb, out_f32=bool(rng.integers(2)))
        m, k, n = (int(v) for v in rng.integers(1, 300, size=3))
        gm.plain_gemm(cfg, f32, m, k, n, 3, False, True, broadcast_a=True)
        gm.plain_gemm(cfg, f32, m, k, n, 2, True, False, broadcast_b=True)


@pytest.mark.parametrize("splits", [2, 3, 7])
def test_split_k_chunks_stay_in_bounds(splits):
    rng = np.random.default_rng(SEED + splits)
    for cfg in [c for c in gm.tile_configs(False) if c.name in ("L8D2", "H", "S", "N", "W")]:
        for _ in range(2):
            m, n = (int(v) for v in rng.integers(1, 400, size=2))
            k = int(rng.integers(129, 3000))
            for ta in (False, True):
                for tb in (False, True):
                    gm.plain_gemm(cfg, False, m, k, n, 1, ta, tb, splits=splits)



def test_column_windows_stay_in_bounds():
    """The two launches of a column remainder (N = 256 q + r, r <= 64): the
    first 256 q columns on the large tiles, the last r on the thin tile with
    and without split K, over odd row pitches and both transpose forms."""
    rng = np.random.default_rng(SEED + 101)
    for f32 in (False, True):
        big = [c for c in gm.tile_configs(f32) if c.name in ("L8D2", "H", "S", "T", "U")]
        thin = [c for c in gm.tile_configs(f32) if c.name == "N"]
        for _ in range(3):
            m = int(rng.integers(65, 700))
            k = int(rng.integers(129, 1200))
            q, r = int(rng.integers(2, 4)), int(rng.choice([1, 3, 8, int(rng.integers(9, 65))]))
            n = 256 * q + r
            for ta in (False, True):
                for tb in (False, True):
                    for cfg in big:
                        gm.window_gemm(cfg, f32, m, k, n, 0, n - r, ta, tb)
                    for cfg in thin:
                        for splits in (1, 3, 6, 16):
                            gm.window_gemm(cfg, f32, m, k, n, n - r, r, ta, tb, splits=splits)
                    if not ta and r <= 8:
                        gm.remainder_rows(f32, m, k, n, n - r, r, tb)
                        # fused with B's re-layout: B read at its source pitch
                        # and dtype (bf16 compute of an fp32 B: autocast)
                        gm.remainder_rows(f32, m, k, n, n - r, r, tb, b_source=True, b_f32=True)
                        gm.remainder_rows(f32, m, k, n, n - r, r, tb, b_source=True, b_f32=f32)

def _counts(rng, groups, total):
    cuts = np.sort(rng.integers(0, total + 1, size=groups - 1))
    counts = np.diff(np.concatenate([[0], cuts, [total]])).tolist()
    counts[int(rng.integers(groups))] = 0  # an expert with no rows
    return counts


@pytest.mark.parametrize("f32", [False, True], ids=["bf16", "fp32"])
def test_grouped_products_stay_in_bounds(f32):
    rng = np.random.default_rng(SEED + 7 + f32)
    e = 4 if f32 else 8
    for cfg in [c for c in gm.tile_configs(f32) if c.name in ("L8D2", "U", "N", "H", "S")]:
        counts = _counts(rng, 5, int(rng.integers(1, 900)))
        inner = e * int(rng.integers(1, 80))
        cols = int(rng.integers(1, 500))
        gm.grouped_gemm(cfg, f32, counts, inner, cols, True)
        # the backward's dY W form reads W as [inner][cols]: 16-byte rows
        gm.grouped_gemm(cfg, f32, counts, inner, (cols + e - 1) // e * e, False)
        with pytest.raises(ValueError):
            gm.grouped_gemm(cfg, f32, counts, inner, e * 3 + 1, False)
        # rows read through the route order (a permutation of token rows)
        tokens = int(sum(counts)) // 2 + 1
        order = rng.integers(0, tokens, size=sum(counts))
        gm.grouped_gemm(cfg, f32, counts, inner, cols, True, gather=order, source_rows=tokens)


@pytest.mark.parametrize("f32", [False, True])
def test_grouped_pair_products_stay_in_bounds(f32):
    rng = np.random.default_rng(SEED + 13 + f32)
    for cfg in [c for c in gm.tile_configs(f32) if c.name in ("L8D2", "U", "N")]:
        counts = _counts(rng, 4, int(rng.integers(1, 700)))
        inner = 64 * int(rng.integers(1, 12))
        cols = 8 * int(rng.integers(1, 60))
        gm.grouped_pair_gemm(cfg, f32, counts, inner, cols, False)
        gm.grouped_pair_gemm(cfg, f32, counts, inner, cols, True)
        with pytest.raises(ValueError):
            gm.grouped_pair_gemm(cfg, f32, counts, inner + 8, cols, False)


def test_swiglu_grouped_and_plain_stay_in_bounds():
    rng = np.random.default_rng(SEED + 11)
    for _ in range(3):
        counts = _counts(rng, 4, int(rng.integers(1, 700)))
        inner = 8 * int(rng.integers(1, 64))
        hidden = int(rng.integers(1, 400))
        gm.grouped_gemm(gm.SWIGLU, False, counts, inner, hidden, True)
        tokens = int(sum(counts)) + 3
        order = rng.integers(0, tokens, size=sum(counts))
        gm.grouped_gemm(gm.SWIGLU, False, counts, inner, hidden, True, gather=order, source_rows=tokens)
        gm.grouped_gemm(gm.SWIGLU, False, [int(rng.integers(1, 600))], inner, hidden, True)  # plain form


@pytest.mark.parametrize("f32", [False, True], ids=["bf16", "fp32"])
def test_grouped_k_products_stay_in_bounds(f32):
    rng = np.random.default_rng(SEED + 13 + f32)
    for cfg in [c for c in gm.tile_configs(f32) if c.name in ("L8D2", "S", "H")]:
        counts = _counts(rng, 6, int(rng.integers(1, 900)))
        rows, cols = (int(v) for v in rng.integers(1, 300, size=2))
        gm.grouped_k_gemm(cfg, f32, counts, rows, cols)


@pytest.mark.parametrize("f32", [False, True], ids=["bf16", "fp32"])
def test_grouped_k_gathered_rows_stay_in_bounds(f32):
    """The weight gradients reading the token rows through the route order
    (GATHER_B, on the two-stage tiles the host maps every choice to): ragged
    groups, empty groups, column counts that are not a multiple of the tile
    and order entries outside the token matrix."""
    rng = np.random.default_rng(SEED + 19 + f32)
    for cfg in [c for c in gm.tile_configs(f32) if c.name in ("L8D2", "T", "U")]:
        counts = _counts(rng, 6, int(rng.integers(1, 900)))
        rows, cols = (int(v) * (4 if f32 else 8) for v in rng.integers(1, 40, size=2))
        tokens = int(sum(counts)) + 5
        order = rng.integers(0, tokens, size=sum(counts))
        gm.grouped_k_gemm(cfg, f32, counts, rows, cols, gather=order, source_rows=tokens)
        if order.size > 3:
            order[:3] = [tokens, -1, (1 << 32) // (cols * (4 if f32 else 2)) + 1]
            gm.grouped_k_gemm(cfg, f32, counts, rows, cols, gather=order, source_rows=tokens)


def test_model_reports_a_gathered_k_index_past_the_source():
    """A planted mistake: the gathered-K kernel without its index check
    issues an order entry past the token rows with its wrapped 32-bit
    offset, which lands on row 1 (2^32 / 128 + 1 rows of 64 bf16)."""
    cfg = gm.tile_configs(False)[0]
    order = np.arange(8)
    gm.grouped_k_gemm(cfg, False, [3, 0, 5], 16, 64, gather=order, source_rows=8)
    order[4] = (1 << 32) // 128 + 1
    gm.grouped_k_gemm(cfg, False, [3, 0, 5], 16, 64, gather=order, source_rows=8)
    with pytest.raises(gm.Violation):
        gm.grouped_k_gemm(cfg, False, [3, 0, 5], 16, 64, gather=order, source_rows=8, index_check=False)


def test_short_k_strips_stay_in_bounds():
    rng = np.random.default_rng(SEED + 17)
    for m, k, n, batch in [(700, 64, 1040, 2), (129, 24, 144, 3), (64, 8, 2064, 1), (2048, 64, 256, 1)]:
        gm.short_strip(m, k, n, batch, 4)
    for _ in range(3):
        m = int(rng.integers(1, 600))
        k = int(rng.integers(1, 65))
        n = 16 * int(rng.integers(1, 70))
        gm.short_strip(m, k, n, int(rng.integers(1, 3)), 4)


def test_pingpong_copies_stay_in_bounds():
    """The ping-pong kernel's copies (descriptor per instruction, range up to
    the operand's end): ragged M and N in every transpose form, odd pitches
    that force the re-layout, broadcast batches; each step fills its LDS
    slot exactly once at OperandTile's coordinates."""
    rng = np.random.default_rng(SEED + 99)
    shapes = [(257, 64, 129), (300, 128, 31), (1, 64, 1), (520, 192, 300)]
    shapes += [(int(rng.integers(1, 600)), 64 * int(rng.integers(1, 5)), int(rng.integers(1, 600))) for _ in range(3)]
    for m, k, n in shapes:
        for ta in (False, True):
            for tb in (False, True):
                gm.pingpong_gemm(m, k, n, 1, ta, tb)
    gm.pingpong_gemm(130, 128, 70, 3, False, True, broadcast_a=True)
    gm.pingpong_gemm(70, 64, 130, 2, True, False, broadcast_b=True)


def test_model_reports_a_pingpong_range_past_the_operand():
    """A planted mistake: copy descriptors that span the tile's 256 rows
    instead of ending at the operand read past the allocation in a ragged
    last tile."""
    gm.pingpong_gemm(300, 64, 40, 1, False, True)
    with pytest.raises(gm.Violation):
        gm.pingpong_gemm(300, 64, 40, 1, False, True, range_rule="tile")


def test_model_reports_a_cut_last_chunk():
    """A planted mistake: an MN-major range that ends at the extent (129
    columns, re-laid out to a pitch of 136) cuts the chunk of columns
    128-135 in the last k-row, so column 128 would read zero."""
    gm.pingpong_gemm(64, 64, 129, 1, False, False)
    with pytest.raises(gm.Violation):
        gm.pingpong_gemm(64, 64, 129, 1, False, False, range_rule="exact")
