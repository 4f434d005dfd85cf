"""Latency table for CostAwareChain on the HIP backend (the reference's
scripts/time_draft_step.py:1-98).

    python -m woodcock_amd.costs --ctx 512 --max-n 7 --sizes 16384 --out costs.json

Measures, with GPU events around captured graphs of the launches a round makes:
  head     final norm + draft head + argmax + d2t on one row (wc_draft_head_norm)
  step     one chain draft step: head + one drafter layer at the context, the
           KV entry rolled back (time_draft_step.py:54-59)
  verify   the target forward over n rows -- embedding, every decoder layer,
           final norm + tied head -- plus the row argmax, n = 1..max_n
           (time_draft_step.py:87-96)
Each figure is the median over `iters` replays.  The result has the
reference's layout, {"ctx", "drafter": {"full" | str(K): {"head_ms",
"step_ms"}}, "verify_ms": {n: ms}}, which CostAwareChain.from_costs reads
(python/woodcock/policies.py:97-101).  Seeded random-init weights of the named
shapes stand in for checkpoints (a drafter directory can be given instead).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json

import numpy as np
import torch

from . import _lib
from .runtime import ptr, stream_ptr


def _capture(fn, reps: int = 1):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    return g


def median_ms(fn, iters: int, warmup: int = 3, reps: int = 8) -> float:
    """Median GPU time of one fn() call: a captured graph of `reps` calls,
    timed per replay and divided by reps, so the replay's own launch latency
    is spread over the calls (the reference times each call in a loop of
    mx.eval's, scripts/time_draft_step.py:39-98)."""
    fn()
    torch.cuda.synchronize()
    g = _capture(fn, reps)
    for _ in range(warmup):
        g.replay()
    ts = []
    for _ in range(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) / reps)
    return float(np.median(ts))


def time_drafter(d, ctx: int, iters: int) -> dict[str, float]:
    """head_ms / step_ms of a Drafter at drafter context ctx."""
    cfg, dev = d.cfg, d.device
    cache = d.make_cache(ctx + 16)
    for c in cache:
        c.keys[0, :, :ctx].normal_()
        c.values[0, :, :ctx].normal_()
    dm = cfg.hidden_size
    dims, W, ws = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws)
    hid = torch.randn(1, dm, device=dev)
    out = torch.empty_like(hid)
    hid2 = torch.empty_like(hid)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    off = torch.tensor([ctx], dtype=torch.int32, device=dev)
    kp = (C.c_void_p * len(cache))(*[c.keys.data_ptr() for c in cache])
    vp = (C.c_void_p * len(cache))(*[c.values.data_ptr() for c in cache])
    kvdt = _lib.WC_BF16 if cache[0].keys.dtype == torch.bfloat16 else _lib.WC_F32

    def head():
        _lib.call("wc_draft_head_norm", dims, W, ptr(hid), dm, None, 0, ptr(out), dm, None, 0, ptr(tok), None, None,
                  ws, stream_ptr())

    def step():
        head()
        _lib.call("wc_drafter_forward", dims, W, ptr(tok), ptr(out), dm, None, 0, 1, None, kp, vp, kvdt,
                  cache[0].capacity, ptr(off), 0, None, None, 0, ptr(hid2), None, None, ws, stream_ptr())

    return {"head_ms": median_ms(head, iters), "step_ms": median_ms(step, iters)}


def time_verify(tm, ctx: int, max_n: int, iters: int) -> dict[int, float]:
    """verify_ms[n] of a TargetModel: the forward over n rows at context ctx plus the argmax."""
    dev = tm.device
    cache = tm.make_cache(ctx + max_n + 8)
    for c in cache:
        c.keys[0, :, :ctx].normal_()
        c.values[0, :, :ctx].normal_()
        c.offset = ctx
    off = torch.tensor([ctx], dtype=torch.int32, device=dev)
    logits = torch.empty(max_n, tm.cfg.vocab_size, device=dev)
    taps = [torch.empty(max_n, tm.cfg.hidden_size, device=dev) for _ in tm.feature_layers]
    am = torch.empty(max_n, dtype=torch.int32, device=dev)
    from .runtime import workspace

    vws = workspace(dev)
    res = {}
    for n in range(1, max_n + 1):
        tok = torch.randint(0, tm.cfg.vocab_size, (n,), dtype=torch.int32, device=dev)

        def verify():
            tm(tok, cache, off, logits=logits[:n], taps=taps)
            _lib.call("wc_argmax_rows", ptr(logits), n, tm.cfg.vocab_size, logits.stride(0), ptr(am), ptr(vws),
                      stream_ptr())

        res[n] = median_ms(verify, iters)
    return res


def measure(drafter_cfg=None, target_cfg=None, ctx: int = 512, sizes=(16384,), max_n: int = 7, iters: int = 50,
            seed: int = 0, drafter_path=None, device="cuda") -> dict:
    from .config import QWEN3_EOS, qwen3_1p7b_drafter
    from .drafter import Drafter
    from .synthetic import draft_vocab
    from .target import TargetConfig, TargetModel, random_target

    dev = torch.device(device)
    dcfg = drafter_cfg or qwen3_1p7b_drafter()
    tcfg = target_cfg or TargetConfig()
    res = {"ctx": ctx, "drafter": {}, "verify_ms": {}}
    for k in [None, *sizes]:
        d = Drafter.load(drafter_path, device=dev) if drafter_path else Drafter.from_synthetic(dcfg, seed=seed,
                                                                                                 device=dev)
        if k is not None:
            d.restrict_vocab(draft_vocab(d.cfg.vocab_size, k, seed=seed, always=QWEN3_EOS))
        res["drafter"]["full" if k is None else str(k)] = time_drafter(d, ctx, iters)
        del d
        torch.cuda.empty_cache()
    tm = TargetModel(tcfg, random_target(tcfg, seed=seed + 1, device=dev), dev, max_rows=max(8, max_n))
    res["verify_ms"] = {str(n): v for n, v in time_verify(tm, ctx, max_n, iters).items()}
    return res


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--drafter", help="drafter directory (config.json + model.safetensors); default: random init")
    ap.add_argument("--sizes", type=int, nargs="*", default=[16384], help="restricted head sizes")
    ap.add_argument("--ctx", type=int, default=512)
    ap.add_argument("--max-n", type=int, default=7)
    ap.add_argument("--iters", type=int, default=50)
    ap.add_argument("--layers", type=int, default=28, help="target decoder layers (Qwen3-1.7B: 28)")
    ap.add_argument("--out")
    a = ap.parse_args(argv)
    from .target import TargetConfig

    res = measure(target_cfg=TargetConfig(num_layers=a.layers), ctx=a.ctx, sizes=a.sizes, max_n=a.max_n,
                  iters=a.iters, drafter_path=a.drafter)
    print(json.dumps(res, indent=1))
    if a.out:
        with open(a.out, "w") as f:
            json.dump(res, f, indent=1)


if __name__ == "__main__":
    main()
