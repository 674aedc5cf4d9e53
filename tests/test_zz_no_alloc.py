"""GPU: di_group_norm_noalloc (partials in the library's static device
scratch instead of the context workspace) against di_group_norm on the same
inputs, bit for bit, on two calls in a row with the second one smaller (the
scratch keeps the first call's contents), for the NCHW fp32 path (cfg1's
[1,320,64,64] GN+SiLU, then [1,64,16,16]) and the NHWC fp16 U-Net path;
a request whose partials exceed the scratch fails cleanly before any launch,
and the library's live-buffer count and workspace size do not move."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NORM_SILU = 1  # DI_NORM_SILU


def _norm(d, fn, x, g, b, N, G, cpg, HW, dt, layout, nbytes):
    import drawinstant
    y = d.create_buffer(nbytes)
    try:
        drawinstant.call(fn, d.ctx, x.handle, g.handle, b.handle, y.handle, N, G, cpg, HW, 1e-5,
                         NORM_SILU, dt, layout)
        d.sync()
        return d.download(y, np.float32 if dt == drawinstant.F32 else np.float16)
    finally:
        y.destroy()


@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
def test_noalloc_matches_group_norm(layout):
    import drawinstant
    d = drawinstant.Device(0)
    try:
        rng = np.random.default_rng(3)
        if layout == "nchw":
            dt, lay, es = drawinstant.F32, drawinstant.NCHW, 4
            # groups of 81920 elements take the two-kernel path (partials in
            # the scratch), then smaller ones the single-launch path
            cases = [(1, 32, 20, 64 * 64), (1, 8, 40, 32 * 64), (1, 32, 10, 64 * 64),
                     (1, 32, 2, 16 * 16)]
        else:
            dt, lay, es = drawinstant.F16, drawinstant.NHWC, 2
            cases = [(2, 32, 20, 32 * 32), (1, 32, 4, 8 * 8)]
        for N, G, cpg, HW in cases:
            C = G * cpg
            n = N * C * HW
            x = d.create_buffer(n * es)
            d.fill_normal(x, n, 11 + N + C, dtype=dt)
            g = d.storage((1 + 0.02 * rng.standard_normal(C)).astype(np.float32))
            b = d.storage((0.02 * rng.standard_normal(C)).astype(np.float32))
            ws0, live0 = d.workspace_stats(), d.pool_stats()["live"]
            got = _norm(d, "di_group_norm_noalloc", x, g, b, N, G, cpg, HW, dt, lay, n * es)
            ws1, live1 = d.workspace_stats(), d.pool_stats()["live"]
            ref = _norm(d, "di_group_norm", x, g, b, N, G, cpg, HW, dt, lay, n * es)
            print(f"[noalloc] {layout} N={N} C={C} HW={HW}: equal={np.array_equal(got, ref)} "
                  f"ws {ws0['bytes']} -> {ws1['bytes']}", flush=True)
            assert np.array_equal(got, ref)
            assert np.isfinite(got.astype(np.float32)).all()
            assert ws1 == ws0 and live1 == live0
            for t in (x, g, b):
                t.destroy()
    finally:
        d.destroy()


def test_noalloc_rejects_oversize():
    """NHWC partials of 4097 images x 32 groups (1 MiB + 2 KiB) exceed the
    static scratch: DI_EUNSUPPORTED with a message, nothing launched."""
    import drawinstant
    from drawinstant.device import DiError
    d = drawinstant.Device(0)
    try:
        N, G, cpg, HW = 4097, 32, 1, 1
        x = d.create_buffer(N * G * HW * 2)
        y = d.create_buffer(N * G * HW * 2)
        g = d.storage(np.ones(G, np.float32))
        b = d.storage(np.zeros(G, np.float32))
        with pytest.raises(DiError, match="static scratch"):
            drawinstant.call("di_group_norm_noalloc", d.ctx, x.handle, g.handle, b.handle,
                             y.handle, N, G, cpg, HW, 1e-5, 0, drawinstant.F16, drawinstant.NHWC)
        d.sync()
        for t in (x, y, g, b):
            t.destroy()
    finally:
        d.destroy()
