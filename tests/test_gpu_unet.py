"""GPU tests of the full SD2.1 U-Net denoise step (di_unet_*, cfg5).

* structure: the library's parameter registry, converted to diffusers
  layout, has exactly diffusers' names and shapes (686 tensors, 865,910,724
  parameters for SD2.1);
* parity: a narrow-channel U-Net of the same architecture against the C-oracle
  composition, and the full SD2.1 step (B=1 and B=4) against the same
  composition on torch float32 with the downloaded weights: rel-L2 <= 1e-2;
* size-independent properties at full size: batch independence, bit-exact
  determinism, graph replay == eager, state_dict round trip.
"""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import unet_ref

pytestmark = pytest.mark.gpu


def _inputs(rng, B, H, W, S, cross):
    x = rng.standard_normal((B, 4, H, W)).astype(np.float32)
    ctx = rng.standard_normal((B, S, cross)).astype(np.float32)
    return x, ctx


@pytest.fixture(scope="module")
def sd21(dev):
    from drawinstant.unet import UNet
    u = UNet(dev, seed=501)
    yield u
    u.destroy()


def test_sd21_registry_matches_diffusers(sd21):
    sd = sd21.state_dict(np.float16)
    shapes = unet_ref.unet_param_shapes(unet_ref.sd21_config())
    assert set(sd) == set(shapes)
    assert all(sd[k].shape == tuple(v) for k, v in shapes.items())
    assert sum(v.size for v in sd.values()) == 865_910_724
    assert all(np.isfinite(v).all() for v in sd.values())


def test_small_unet_vs_oracle(dev, rng):
    from drawinstant.unet import UNet, UNetConfig
    cfg = UNetConfig.small()
    u = UNet(dev, cfg, seed=7)
    try:
        x, ctx = _inputs(rng, 1, 16, 16, 77, cfg.cross_dim)
        got = u(x, 999.0, ctx)
        ref = unet_ref.unet_forward(unet_ref.OracleOps(), u.state_dict(), cfg.as_dict(), x,
                                    np.array([999.0], np.float32), ctx)
        err = rel_l2(got, ref)
        print(f"[small unet] rel-L2 {err:.2e} max-abs {np.max(np.abs(got - ref)):.2e}", flush=True)
        assert np.isfinite(got).all() and err <= 1e-2
    finally:
        u.destroy()


def test_small_unet_narrow_tile_vs_oracle(dev, rng, monkeypatch):
    """Every GEMM / conv of a step on the 64 x 32 tile (DI_GEMM_TILE=14):
    the transformers' projections write row statistics of their outputs per
    32-column tile, twice the pairs of a 64-column tile, into the
    [rows][ceil(N / 32)] buffer, and the folded LayerNorms read them; the
    step matches the oracle composition."""
    from drawinstant.unet import UNet, UNetConfig
    monkeypatch.setenv("DI_GEMM_TILE", "14")
    cfg = UNetConfig.small()
    u = UNet(dev, cfg, seed=7)
    try:
        x, ctx = _inputs(rng, 1, 16, 16, 77, cfg.cross_dim)
        got = u(x, 999.0, ctx)
        ref = unet_ref.unet_forward(unet_ref.OracleOps(), u.state_dict(), cfg.as_dict(), x,
                                    np.array([999.0], np.float32), ctx)
        err = rel_l2(got, ref)
        print(f"[small unet, 64x32 tile] rel-L2 {err:.2e}", flush=True)
        assert np.isfinite(got).all() and err <= 1e-2
    finally:
        u.destroy()


@pytest.mark.parametrize("var,tol", [("DI_CONV_IN_DIRECT", 5e-4)])
@pytest.mark.parametrize("B,H,W", [(1, 16, 16), (2, 8, 24)])
def test_edge_convs_direct_match_implicit_gemm(dev, rng, monkeypatch, var, tol, B, H, W):
    """The direct conv_in kernel (NCHW fp32 latent in, GroupNorm statistics
    out) against the layout pass + implicit-GEMM conv it replaces, over a
    whole narrow U-Net step, and both against the oracle.  Both round the
    latent to fp16 and accumulate in fp32, in another order, so they agree
    to rounding, not bit for bit."""
    from drawinstant.unet import UNet, UNetConfig
    cfg = UNetConfig.small()
    u = UNet(dev, cfg, seed=7)
    try:
        x, ctx = _inputs(rng, B, H, W, 77, cfg.cross_dim)
        got = {}
        for flag in ("0", "1"):
            monkeypatch.setenv(var, flag)
            got[flag] = u(x, 999.0, ctx)
        ref = unet_ref.unet_forward(unet_ref.OracleOps(), u.state_dict(), cfg.as_dict(), x,
                                    np.full(B, 999.0, np.float32), ctx)
        d, e0, e1 = rel_l2(got["1"], got["0"]), rel_l2(got["0"], ref), rel_l2(got["1"], ref)
        print(f"[{var}] B={B} {H}x{W}: direct vs implicit GEMM {d:.2e}, vs oracle "
              f"{e1:.2e} (implicit GEMM {e0:.2e})", flush=True)
        assert np.isfinite(got["1"]).all() and d <= tol and e1 <= 1e-2
    finally:
        u.destroy()


def test_layer_norm_fold_follows_uploads(dev, rng):
    """The transformer LayerNorms (norm1/2/3) run inside their projections'
    GEMMs, on weights derived from the parameters (W * gamma, beta . W + bias)
    the first time the U-Net runs after a parameter upload.  Strong gammas /
    betas uploaded after a first step (so the derived weights must be
    refreshed) still give the oracle's result; with the near-identity
    initial affines a dropped beta term or a stale derivation would pass."""
    import re
    from drawinstant.unet import UNet, UNetConfig
    cfg = UNetConfig.small()
    u = UNet(dev, cfg, seed=11)
    try:
        x, ctx = _inputs(rng, 1, 16, 16, 77, cfg.cross_dim)
        first = u(x, 999.0, ctx)  # derives the folded weights
        sd = u.state_dict(np.float32)
        pat = re.compile(r"transformer_blocks\.0\.norm[123]\.(weight|bias)$")
        for k in sd:
            m = pat.search(k)
            if m:
                n = rng.standard_normal(sd[k].shape).astype(np.float32)
                sd[k] = (1.0 + 0.5 * n) if m.group(1) == "weight" else 0.5 * n
        u.load_state_dict(sd)
        got = u(x, 999.0, ctx)
        ref = unet_ref.unet_forward(unet_ref.OracleOps(), u.state_dict(), cfg.as_dict(), x,
                                    np.array([999.0], np.float32), ctx)
        err = rel_l2(got, ref)
        print(f"[ln fold] rel-L2 {err:.2e}, change from the first step {rel_l2(got, first):.2e}",
              flush=True)
        assert np.isfinite(got).all() and err <= 1e-2
        assert rel_l2(got, first) > 5e-2  # the new affines took effect
    finally:
        u.destroy()


def _torch_ref(sd21, x, t, ctx):
    sd = sd21.state_dict(np.float32)
    out = unet_ref.unet_forward(unet_ref.TorchOps("cuda"), sd, sd21.config.as_dict(), x,
                                np.asarray(t, np.float32), ctx)
    return out.cpu().numpy()


def test_sd21_step_b1_vs_torch_fp32(sd21, rng):
    """cfg5 at B=1: latent [1,4,64,64], context [1,77,1024], timestep 999."""
    x, ctx = _inputs(rng, 1, 64, 64, 77, 1024)
    got = sd21(x, 999.0, ctx)
    ref = _torch_ref(sd21, x, [999.0], ctx)
    err = rel_l2(got, ref)
    print(f"[sd21 B=1] rel-L2 {err:.2e} max-abs {np.max(np.abs(got - ref)):.2e} "
          f"|ref| max {np.abs(ref).max():.2f}", flush=True)
    assert np.isfinite(got).all() and err <= 1e-2


def test_sd21_step_b4_batch_independent(sd21, rng):
    """cfg5 at B=4 (different timesteps): each sample equals its B=1 step, and
    the batch matches the torch fp32 reference."""
    x, ctx = _inputs(rng, 4, 64, 64, 77, 1024)
    ts = np.array([999.0, 500.0, 250.0, 1.0], np.float32)
    got = sd21(x, ts, ctx)
    for b in (0, 3):
        one = sd21(x[b:b + 1], ts[b], ctx[b:b + 1])
        # B=4 and B=1 tile the GEMMs differently (M = 4*HW vs HW), so fp32
        # summation order and the fp16 roundings of ~50 layers differ: ~2e-3
        # measured.  Mixing samples (GN stats, attention, temb across the
        # batch) would be an O(1) error.
        assert rel_l2(got[b:b + 1], one) <= 5e-3
    err = rel_l2(got, _torch_ref(sd21, x, ts, ctx))
    print(f"[sd21 B=4] rel-L2 {err:.2e}", flush=True)
    assert err <= 1e-2


def test_sd21_gn_in_reducers_matches_separate(sd21, rng, monkeypatch):
    """cfg5 at B=1 with the GroupNorms that split-K reducers apply (each
    ResNet's GN2 in conv1's reducer; a transformer's GN in the conv2 reducer
    of the ResNet before it) against the same step with every GroupNorm as
    its own apply launch (DI_GN_REDUCE_FUSE=0).  The fp16 values the
    GroupNorms read are the same; only the fp32 summation order of their
    statistics differs."""
    x, ctx = _inputs(rng, 1, 64, 64, 77, 1024)
    fused = sd21(x, 999.0, ctx)
    monkeypatch.setenv("DI_GN_REDUCE_FUSE", "0")
    sep = sd21(x, 999.0, ctx)
    err = rel_l2(fused, sep)
    print(f"[sd21 gn reducers] rel-L2 {err:.2e} max-abs {np.max(np.abs(fused - sep)):.2e}",
          flush=True)
    # measured 1.4e-3: rounding differences carried through ~50 fp16 layers,
    # the same size as the whole step's distance to fp32 (1.7e-3); a wrong
    # group, channel or statistic would be O(1)
    assert np.isfinite(fused).all() and err <= 5e-3


def test_sd21_gn_exchange_reducers(sd21, rng, monkeypatch):
    """cfg5 at B=4 and B=1: the 16 x 16 and 32 x 32 split-K reducers that apply a
    GroupNorm with four or eight workgroups per (group, image) exchanging
    their statistics give the
    same bits when every workgroup recomputes the other slices' sums itself
    (DI_GN_XCHG_SPIN=0, the path a workgroup takes when a slice does not
    arrive), and agree with one workgroup per group or a separate apply
    launch (DI_GN_REDUCE_XCHG=0) up to the fp32 summation order."""
    x4, ctx4 = _inputs(rng, 4, 64, 64, 77, 1024)
    t4 = np.array([999.0, 750.0, 500.0, 250.0], np.float32)
    b4 = sd21(x4, t4, ctx4)  # four images: four records per group
    monkeypatch.setenv("DI_GN_XCHG_SPIN", "0")
    np.testing.assert_array_equal(sd21(x4, t4, ctx4), b4)
    monkeypatch.delenv("DI_GN_XCHG_SPIN")
    x, ctx = _inputs(rng, 1, 64, 64, 77, 1024)
    xch = sd21(x, 999.0, ctx)
    monkeypatch.setenv("DI_GN_XCHG_SPIN", "0")
    rec = sd21(x, 999.0, ctx)
    monkeypatch.delenv("DI_GN_XCHG_SPIN")
    np.testing.assert_array_equal(rec, xch)
    monkeypatch.setenv("DI_GN_REDUCE_XCHG", "0")
    one = sd21(x, 999.0, ctx)
    monkeypatch.delenv("DI_GN_REDUCE_XCHG")
    err = rel_l2(xch, one)
    print(f"[sd21 gn exchange] rel-L2 {err:.2e} vs one workgroup per group", flush=True)
    assert np.isfinite(xch).all() and err <= 5e-3
    np.testing.assert_array_equal(sd21(x, 999.0, ctx), xch)


def test_sd21_shortcut_partials_match_separate(sd21, rng, monkeypatch):
    """cfg5 at B=1 with each split-K ResNet shortcut's partials summed by its
    conv2's reducer (with the summed bias) against the same step with the
    shortcut as its own GEMM + reducer writing an fp16 tensor that conv2
    adds (DI_SK_PARTIALS=0).  The two differ by that tensor's fp16 rounding
    and the order of the fp32 sums."""
    x, ctx = _inputs(rng, 1, 64, 64, 77, 1024)
    fused = sd21(x, 999.0, ctx)
    monkeypatch.setenv("DI_SK_PARTIALS", "0")
    sep = sd21(x, 999.0, ctx)
    err = rel_l2(fused, sep)
    print(f"[sd21 shortcut partials] rel-L2 {err:.2e} max-abs {np.max(np.abs(fused - sep)):.2e}",
          flush=True)
    # measured 1.4e-3 (see the GroupNorm comparison above)
    assert np.isfinite(fused).all() and err <= 5e-3


def test_sd21_step_b2_batch_independent(sd21, rng):
    """cfg5 at B=2 (the largest batch whose time_emb_proj GEMV rides in the
    first GroupNorm's launch; every split-K reducer's GroupNorm runs one
    workgroup row per image): each sample equals its B=1 step."""
    x, ctx = _inputs(rng, 2, 64, 64, 77, 1024)
    ts = np.array([999.0, 250.0], np.float32)
    got = sd21(x, ts, ctx)
    for b in (0, 1):
        one = sd21(x[b:b + 1], ts[b], ctx[b:b + 1])
        err = rel_l2(got[b:b + 1], one)
        print(f"[sd21 B=2] sample {b} vs B=1 rel-L2 {err:.2e}", flush=True)
        assert np.isfinite(got[b:b + 1]).all() and err <= 5e-3


def test_sd21_graph_replay_matches_eager(dev, sd21, rng):
    """Eager twice is bit-identical; the captured graph replayed several times,
    with eager work and synchronisation in between, matches eager exactly."""
    x, ctx = _inputs(rng, 1, 64, 64, 77, 1024)
    bs, bt, bc = dev.storage(x), dev.storage(np.array([999.0], np.float32)), dev.storage(ctx)
    bo = dev.create_buffer(x.nbytes)
    sd21.forward(bs, bt, bc, bo)
    eager = dev.download(bo, np.float32, x.shape)
    sd21.forward(bs, bt, bc, bo)
    np.testing.assert_array_equal(dev.download(bo, np.float32, x.shape), eager)
    for _ in range(3):
        dev.fill_normal(bo, x.size, 9)  # clobber the output between replays
        sd21.forward(bs, bt, bc, bo, graph=True)
        dev.sync()
        np.testing.assert_array_equal(dev.download(bo, np.float32, x.shape), eager)
        sd21(x, 999.0, ctx)  # unrelated eager step in between
    for b in (bs, bt, bc, bo):
        b.destroy()


def test_graph_replay_survives_workspace_growth(rng):
    """A captured U-Net graph keeps addressing the workspace it was captured
    with: growing the context workspace afterwards (a large split-K linear)
    retires the old allocation instead of freeing it, the replay stays
    bit-identical to eager, and dropping the graph frees the retired block."""
    import drawinstant
    from drawinstant.unet import UNet, UNetConfig
    d = drawinstant.Device(0)  # fresh context: its workspace starts empty
    try:
        cfg = UNetConfig.small()
        u = UNet(d, cfg, seed=11)
        x, ctx = _inputs(rng, 1, 16, 16, 77, cfg.cross_dim)
        bs, bt, bc = d.storage(x), d.storage(np.array([999.0], np.float32)), d.storage(ctx)
        bo = d.create_buffer(x.nbytes)
        shape = dict(B=1, H=16, W=16, Sctx=77)
        u.forward(bs, bt, bc, bo, **shape)
        eager = d.download(bo, np.float32, x.shape)
        u.forward(bs, bt, bc, bo, graph=True, **shape)
        d.sync()
        np.testing.assert_array_equal(d.download(bo, np.float32, x.shape), eager)
        ws0 = d.workspace_stats()
        print(f"[ws] after capture {ws0}", flush=True)
        assert ws0["pinned"] == 1 and ws0["retired"] == 0 and ws0["bytes"] > 0
        # M = 64 rows against a long K: the planner splits K, and the fp32
        # partials (splits x 64 x N x 4 bytes) outgrow the captured workspace
        M, N = 64, 2560
        grown = None
        for K in (8192, 32768):
            xa = d.create_buffer(M * K * 2)
            wa = d.create_buffer(N * K * 2)
            ya = d.create_buffer(M * N * 2)
            d.fill_normal(xa, M * K, 3, dtype=drawinstant.F16)
            d.fill_normal(wa, N * K, 4, std=0.01, dtype=drawinstant.F16)
            drawinstant.call("di_linear", d.ctx, xa.handle, wa.handle, 0, 0, ya.handle, M, N, K, 0,
                             drawinstant.F16)
            d.sync()
            for b in (xa, wa, ya):
                b.destroy()
            grown = d.workspace_stats()
            print(f"[ws] after linear K={K}: {grown}", flush=True)
            if grown["bytes"] > ws0["bytes"]:
                break
        assert grown["bytes"] > ws0["bytes"], "the split-K linear did not grow the workspace"
        assert grown["retired"] == 1 and grown["pinned"] == 1
        for _ in range(2):
            d.fill_normal(bo, x.size, 9)
            u.forward(bs, bt, bc, bo, graph=True, **shape)
            d.sync()
            np.testing.assert_array_equal(d.download(bo, np.float32, x.shape), eager)
        u.destroy()
        after = d.workspace_stats()
        assert after["retired"] == 0 and after["pinned"] == 0
        for b in (bs, bt, bc, bo):
            b.destroy()
    finally:
        d.destroy()


def test_graph_check_denoise_loop(dev, sd21, rng, monkeypatch):
    """DI_GRAPH_CHECK=1 over the SD2.1 denoise loop (graph replays between
    on-device copies of the timestep and scheduler kernels, as bench.py's
    denoise leg runs it): every node of the captured step is a kernel launch
    with an in-range grid / block / LDS size, and before every replay the
    graph's workspace, scratch buffers and I/O buffers are still its own.
    The looped result equals the eager loop bit for bit."""
    from drawinstant import scheduler as S
    monkeypatch.setenv("DI_GRAPH_CHECK", "1")
    ctx = rng.standard_normal((1, 77, 1024)).astype(np.float32)
    bc = dev.storage(ctx)
    lat = dev.create_buffer(4 * 64 * 64 * 4)
    d = S.Denoiser(sd21, steps=4)
    try:
        d.run(bc, lat, seed=3, graph=False)
        eager = dev.download(lat, np.float32)
        for _ in range(3):
            d.run(bc, lat, seed=3, graph=True)
            dev.sync()
            np.testing.assert_array_equal(dev.download(lat, np.float32), eager)
    finally:
        d.destroy()
        for b in (bc, lat):
            b.destroy()


def test_state_dict_round_trip(dev):
    from drawinstant.unet import UNet, UNetConfig
    cfg = UNetConfig.small()
    a, b = UNet(dev, cfg, seed=1), UNet(dev, cfg, seed=2)
    try:
        sa = a.state_dict(np.float16)
        b.load_state_dict(sa)
        sb = b.state_dict(np.float16)
        assert set(sa) == set(sb)
        for k in sa:
            np.testing.assert_array_equal(sa[k], sb[k])
    finally:
        a.destroy()
        b.destroy()


def test_unet_forward_hip_entry_point(sd21, rng):
    """unetForwardWGSL counterpart: integer-rounded timestep, host arrays in
    and out; equals UNet.forward on the same (seed 0) weights."""
    from drawinstant import unet as U
    x, ctx = _inputs(rng, 1, 64, 64, 77, 1024)
    res = U.unet_forward_hip(x, 998.6, ctx)
    assert res["dims"] == [1, 4, 64, 64] and res["ms"] > 0
    dev, u = U._state["unet"]
    direct = u(x, 999.0, ctx)
    np.testing.assert_array_equal(res["out"], direct)
