"""Measure the best GEMM tile / split-K choice for every GEMM shape of one
SD2.1 U-Net step (or one 512x512 VAE decode) and write them as
gemm_tuned.inc (the table gemm_plan consults before its cost model).

    python draw-instant_amd/csrc/gemm_tune.py [--model unet|vae] [--append]
                                              [--out PATH] [--iters N]

--append keeps the table's existing rows and adds the shapes it lacks (so
the VAE's shapes join the U-Net's).  Needs the GPU and a built
libdrawinstant_hip.so.  Steps:
  1. one eager U-Net step (VAE decode) with DI_TRACE_GEMM=1 lists its GEMM
     calls;
  2. each distinct shape (M, N, K, conv geometry, GEGLU) is re-issued as a
     di_linear / di_conv2d call and timed for every (tile, splits) pair with
     DI_GEMM_TILE / DI_GEMM_SPLITS forcing the plan;
  3. weights rotate over copies totalling > 256 MiB (the MI355X MALL size),
     so B streams from HBM as in the step, where each weight is read once.
Ties within 3% go to the smaller split factor (less workspace traffic).
"""
import argparse
import os
import re
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # draw-instant_amd/

TILES = (0, 1, 2, 3, 5, 6, 7, 8, 9, 10, 11, 12)  # TILE_128x160 (4) is not built
SPLITS = (1, 2, 3, 4, 6, 8, 12, 16)
TRACE_RE = re.compile(r"\[di_gemm\] (.*)")


def trace_step(model="unet"):
    """GEMM calls of one eager 512x512 step / decode (trace lines go to fd 2)."""
    import numpy as np
    os.environ["DI_TRACE_GEMM"] = "1"
    import drawinstant
    from drawinstant.unet import UNet
    from drawinstant.vae import VAE
    fd, path = tempfile.mkstemp(suffix=".log")
    saved = os.dup(2)
    os.dup2(fd, 2)
    try:
        dev = drawinstant.Device(0)
        rng = np.random.default_rng(0)
        x = rng.standard_normal((1, 4, 64, 64)).astype(np.float32)
        if model == "vae":
            v = VAE(dev, seed=1)
            v(x, graph=False)
            dev.sync()
            v.destroy()
        else:
            u = UNet(dev, seed=1)
            ctx = rng.standard_normal((1, 77, 1024)).astype(np.float32)
            u(x, 999.0, ctx, graph=False)
            dev.sync()
            u.destroy()
        dev.destroy()
    finally:
        os.dup2(saved, 2)
        os.close(saved)
        os.close(fd)
    calls = []
    for line in open(path):
        m = TRACE_RE.search(line)
        if m:
            calls.append(dict(kv.split("=") for kv in m.group(1).split()))
    os.unlink(path)
    return calls


def key_of(c):
    conv = int(c["amode"]) != 0
    return (int(c["M"]), int(c["N"]), int(c["K"]), int(conv), int(c["ks"]) if conv else 0,
            int(c["stride"]) if conv else 0, int(c["up"]) if conv else 0,
            int(int(c["act"]) == 2))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=os.path.join(HERE, "gemm_tuned.inc"))
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--model", choices=("unet", "vae"), default="unet")
    ap.add_argument("--append", action="store_true")
    args = ap.parse_args()
    kept = []
    if args.append and os.path.exists(args.out):
        kept = [ln for ln in open(args.out) if ln.startswith("{")]
    have = {tuple(int(v) for v in ln[1:ln.index("}")].split(",")[:8]) for ln in kept}
    calls = trace_step(args.model)
    os.environ.pop("DI_TRACE_GEMM", None)
    shapes = {}
    for c in calls:
        if c["elem"] != "1" or c["fast"] != "1":
            continue
        k = key_of(c)
        if k in have:
            continue
        shapes.setdefault(k, [c, 0])[1] += 1
    print(f"[tune] {len(calls)} GEMM calls, {len(shapes)} distinct fast fp16 shapes", flush=True)

    import numpy as np
    import drawinstant
    from drawinstant.device import call
    dev = drawinstant.Device(0)
    rng = np.random.default_rng(0)

    # A ~1 ms GEMM queued ahead of each timed batch: the host enqueues the
    # batch while it runs, so the timed kernels run back to back and the
    # measurement is GPU time, not launch overhead.
    nb = 4096
    bx, bw, by = (dev.create_buffer(nb * nb * 2) for _ in range(3))
    dev.fill_normal(bx, nb * nb, 1, dtype=1)
    dev.fill_normal(bw, nb * nb, 2, std=0.02, dtype=1)

    def blocker():
        for _ in range(4):
            call("di_linear", dev.ctx, bx.handle, bw.handle, 0, 0, by.handle, nb, nb, nb, 0, 1)

    def t_us(fn, it):
        fn()
        dev.sync()
        blocker()
        dev.timer_begin(0)
        for _ in range(it):
            fn()
        dev.timer_end(0)
        return dev.timer_ms(0) / it * 1e3

    rows = []
    for k, (c, count) in sorted(shapes.items(), key=lambda kv: -kv[1][1]):
        M, N, K, conv, ks, stride, up, geglu = k
        if conv:
            cin = int(c["cin"])
            h, w = (int(v) for v in c["hw"].split("x"))
            x = dev.storage(rng.standard_normal((1, h, w, cin)).astype(np.float16))
            wbytes = N * ks * ks * cin * 2
        else:
            x = dev.storage(rng.standard_normal((M, K)).astype(np.float16))
            wbytes = N * K * 2
        copies = max(1, min(64, (300 << 20) // wbytes + 1))
        ws = []
        for i in range(copies):
            wb = dev.create_buffer(wbytes)
            dev.fill_normal(wb, wbytes // 2, 100 + i, std=0.02, dtype=1)
            ws.append(wb)
        nout = N // 2 if geglu else N
        y = dev.create_buffer(M * nout * 2)
        state = {"i": 0}

        def fn():
            wb = ws[state["i"] % copies]
            state["i"] += 1
            if conv:
                pad = ks // 2
                call("di_conv2d", dev.ctx, x.handle, wb.handle, 0, 0, y.handle, 1, cin, N, h, w,
                     ks, stride, pad, 2 if up == 2 else 0, 1, 1)
            else:
                call("di_linear", dev.ctx, x.handle, wb.handle, 0, 0, y.handle, M, N, K,
                     2 if geglu else 0, 1)

        best = None
        for tile in TILES:
            if geglu and tile == 5:
                continue
            for sp in SPLITS:
                if sp > 1 and ((K + sp - 1) // sp + 63) // 64 * 64 < 256:
                    break
                if sp > 2 and M >= 65536:  # thousands of tiles already
                    break
                os.environ["DI_GEMM_TILE"] = str(tile)
                os.environ["DI_GEMM_SPLITS"] = str(sp)
                us = t_us(fn, args.iters)
                if best is None or us < best[0] * 0.97 or (us < best[0] and sp <= best[2]):
                    best = (us, tile, sp)
        os.environ.pop("DI_GEMM_TILE", None)
        os.environ.pop("DI_GEMM_SPLITS", None)
        auto = t_us(fn, args.iters)
        print(f"[tune] {k} x{count}: model {auto:7.2f} us, best tile {best[1]} splits {best[2]} "
              f"{best[0]:7.2f} us", flush=True)
        rows.append((k, best[1], best[2], best[0], auto, count))
        for b in ws + [x, y]:
            b.destroy()

    with open(args.out, "w") as f:
        f.write("// Measured GEMM plans for the SD2.1 U-Net step and VAE decode shapes (MI355X),\n")
        f.write("// written by\n")
        f.write("//   python draw-instant_amd/csrc/gemm_tune.py [--model vae --append]\n")
        f.write("// {M, N, K, conv, ks, stride, up, geglu, tile, splits},"
                "  // best us / cost-model us, calls per step\n")
        for ln in kept:
            f.write(ln)
        for (M, N, K, conv, ks, stride, up, geglu), tile, sp, us, auto, count in rows:
            f.write(f"{{{M}, {N}, {K}, {conv}, {ks}, {stride}, {up}, {geglu}, {tile}, {sp}}},"
                    f"  // {us:.2f} / {auto:.2f} us, x{count}\n")
    saved = sum((a - b) * n for _, _, _, b, a, n in rows)
    print(f"[tune] wrote {args.out}: {len(rows)} shapes, {saved:.0f} us per step below the model",
          flush=True)


if __name__ == "__main__":
    main()
