"""The column reduction's entry point that allocates nothing
(adhip_reduce_cols_noalloc, scratch in a static device array) against the
allocating one (adhip_reduce_cols) through the C ABI: bit-identical
results on two calls in a row, the second smaller, for SUM and MAX, both
checked against float64 numpy too.  Collected last (its name), so a
failure here hides no other test.  The split below restates the library's
chunk policy so the test can assert that every call really uses scratch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 1 << 18


def _split(rows, cols):
    blocks = -(-cols // 64)
    split = 1
    while blocks * split < 512 and split < 128 and rows // (2 * split) >= 64:
        split *= 2
    return split


@pytest.fixture
def ctx():
    from ad_amd.device.hip.runtime import Context
    c = Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("op", [0, 1])
def test_noalloc_matches_allocating_entry_point(ctx, op):
    calls = [(16384, 1024), (3000, 100)]          # the second smaller (and not float4-aligned)
    size = max(r * c for r, c in calls)
    x_off, a_off = 0, 4 * size
    b_off = a_off + 4 * 4096
    ctx.reserve(b_off + 4 * 4096)
    rng = np.random.default_rng(7)
    for rows, cols in calls:
        assert _split(rows, cols) > 1 and _split(rows, cols) * cols <= SCRATCH_FLOATS
        print(f"reduce_cols op={op} rows={rows} cols={cols} split={_split(rows, cols)}", flush=True)
        x = rng.standard_normal((rows, cols), dtype=np.float32)
        ctx.write(x_off, x)
        ctx.reduce_cols(x_off, a_off, rows, cols, op)
        ctx.reduce_cols_noalloc(x_off, b_off, rows, cols, op)
        a = np.empty(cols, np.float32)
        b = np.empty(cols, np.float32)
        ctx.read(a_off, a)
        ctx.read(b_off, b)
        assert np.array_equal(a, b)
        if op == 0:
            want = x.astype(np.float64).sum(0)
            bound = np.sqrt(rows) * 4 * np.finfo(np.float32).eps * np.abs(x).astype(np.float64).sum(0)
            assert np.all(np.abs(a - want) <= bound)
        else:
            assert np.array_equal(a, x.max(0))


def test_noalloc_rejects_bad_arguments(ctx):
    ctx.reserve(1 << 20)
    rc = ctx.lib.adhip_reduce_cols_noalloc(ctx.h, ctx.base, ctx.base + 4096, 64, 16, 2)
    assert rc != 0 and b"op must be" in ctx.lib.adhip_last_error(ctx.h)
    rc = ctx.lib.adhip_reduce_cols_noalloc(ctx.h, ctx.base, ctx.base + 4096, 0, 16, 0)
    assert rc != 0 and b"0 rows" in ctx.lib.adhip_last_error(ctx.h)
