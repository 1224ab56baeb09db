"""Writes the golden fixtures of the expert path with the reference xiaotu-moe
CPU engine (``MOE_V2::forward_many``, compiled from the reference's own
headers into ``oracle/_ref`` by ``oracle/build_ref.sh``).

Each fixture is data only: the recipe of its weights (seed, shapes, format --
``tests/helpers.make_dense_layer`` regenerates them bit-identically from the
seed, a SHA-256 of the quantised bytes guards against drift), the routing and
the bf16 tokens as given to the engine, and the engine's fp32 output.

Run from the repository root (needs the reference build):
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "vllm-xtu-moe_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle  # noqa: E402
from helpers import dense_to_numpy, make_dense_layer, random_routing  # noqa: E402
from xtu_moe_amd import formats as F  # noqa: E402

# name -> recipe.  E counts routed experts; the engine sees shared experts as
# extra columns of weight 1.
CASES = {
    # tiny Mixtral-style bf16 layer (H=1024, 8 experts, I=2048, softmax top-2
    # renormalised, router weights N(0, 0.02)); first 16 of the 128 tokens
    "mixtral_tiny_bf16": dict(fmt=F.FMT_BF16, E=8, NS=0, H=1024, I=2048, T=16, K=2, seed=0,
                              router="mixtral", limit=0.0),
    "small_bf16": dict(fmt=F.FMT_BF16, E=8, NS=1, H=512, I=256, T=6, K=2, seed=11, limit=0.0),
    "small_fp8": dict(fmt=F.FMT_FP8, E=8, NS=1, H=512, I=256, T=6, K=2, seed=12, limit=0.0),
    "small_mxfp4": dict(fmt=F.FMT_MXFP4, E=8, NS=1, H=512, I=256, T=6, K=2, seed=13, limit=7.0),
    "small_nvfp4": dict(fmt=F.FMT_NVFP4, E=8, NS=1, H=512, I=256, T=6, K=2, seed=14, limit=7.0),
    # INT8-activation x FP4-code ALIGN path of the engine (MXFP4, e8m0 spread <= 3)
    "small_mxfp4_int8": dict(fmt=F.FMT_MXFP4, E=8, NS=1, H=512, I=256, T=6, K=2, seed=15,
                             limit=7.0, int8=True),
    # the SwiGLU-OAI activation: sigmoid scale alpha and the +beta on `up`
    # (the engine's swiglu_alpha / swiglu_beta) with the clamp at 7
    "small_mxfp4_oai": dict(fmt=F.FMT_MXFP4, E=8, NS=1, H=512, I=256, T=6, K=2, seed=16,
                            limit=7.0, alpha=1.702, beta=1.0),
    "small_fp8_oai": dict(fmt=F.FMT_FP8, E=8, NS=1, H=512, I=256, T=6, K=2, seed=17,
                          limit=7.0, alpha=1.702, beta=1.0),
    "small_mxfp4_int8_oai": dict(fmt=F.FMT_MXFP4, E=8, NS=1, H=512, I=256, T=6, K=2, seed=18,
                                 limit=7.0, alpha=1.702, beta=1.0, int8=True),
    # the ALIGN path where the engine's offset guard (cmin + emin - 128 >= -24,
    # moe_v2_packed4_w4a8.inc:436,1361) fails on every tile: weights N(0,
    # 0.02 * 2^-16), tokens N(0, 2^-24), so the engine computes these tiles in
    # fp32 while the GPU's per-row-scaled int32 path takes them in INT8
    "small_mxfp4_int8_g2": dict(fmt=F.FMT_MXFP4, E=8, NS=1, H=512, I=256, T=6, K=2, seed=19,
                                limit=7.0, int8=True, std=0.02 * 2.0 ** -16, x_scale=2.0 ** -12),
}


def act_args(c: dict) -> dict:
    """The activation parameters of a case (limit, alpha, beta)."""
    return dict(limit=c["limit"], alpha=c.get("alpha", 1.0), beta=c.get("beta", 0.0))


def weights_digest(d: dict) -> str:
    h = hashlib.sha256()
    for k in ("w13", "s13", "gs13", "w2", "s2", "gs2"):
        v = d[k]
        if v is not None:
            h.update(np.ascontiguousarray(v).tobytes())
    return h.hexdigest()


def case_inputs(c: dict):
    """Routing and tokens of a case (numpy, seeded)."""
    import torch

    rng = np.random.default_rng(c["seed"] + 100)
    x = rng.standard_normal((c["T"], c["H"])).astype(np.float32) * np.float32(c.get("x_scale", 1.0))
    x_bits = oracle.f32_to_bf16_bits(x)
    if c.get("router") == "mixtral":
        g = torch.Generator().manual_seed(c["seed"] + 7)
        wr = (torch.randn((c["E"], c["H"]), generator=g) * 0.02).numpy()
        logits = (oracle.bf16_bits_to_f32(x_bits) @ wr.T).astype(np.float32)
        ids, wts = oracle.route_softmax_topk(logits, c["K"])
    else:
        ids, wts = random_routing(c["T"], c["K"], c["E"], seed=c["seed"] + 200, invalid_frac=0.1,
                                  zero_frac=0.1)
    return x_bits, ids, wts


def main(names=None):
    if not oracle.ref_available():
        raise SystemExit("reference engine build (oracle/_ref) missing: run oracle/build_ref.sh")
    L = oracle.ref_lib()
    for name, c in CASES.items():
        if names and name not in names:
            continue
        d = dense_to_numpy(c["fmt"], make_dense_layer(c["fmt"], c["E"] + c["NS"], c["H"], c["I"],
                                                      seed=c["seed"], std=c.get("std", 0.02)))
        x_bits, ids, wts = case_inputs(c)
        T, K, E, NS = c["T"], c["K"], c["E"], c["NS"]
        # the engine takes the shared experts as always-on columns of weight 1 and
        # skips invalid ids / zero weights itself
        eids = ids.astype(np.int64)
        eids = np.where((eids < 0) | (eids >= E), E + NS + 5, eids)   # out of range -> ignored
        if NS:
            eids = np.concatenate([eids, np.tile(np.arange(E, E + NS), (T, 1))], 1)
            ew = np.concatenate([wts, np.ones((T, NS), np.float32)], 1)
        else:
            ew = wts
        eng = oracle.RefEngine(c["fmt"], E + NS, K + NS, c["H"], c["I"], d["w13"], d["s13"],
                               d["w2"], d["s2"], d["gs13"], d["gs2"], **act_args(c))
        if c.get("int8"):
            L.xref_set_int8(1, 1 << 30)
        out = eng.forward(x_bits, eids.astype(np.uint32), ew.astype(np.float32))
        if c.get("int8"):
            L.xref_set_int8(0, 0)
        eng.close()
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), x_bits=x_bits, ids=ids, wts=wts,
                            out=out, digest=np.array(weights_digest(d)),
                            isa=np.array(int(L.xref_isa())))
        print(f"{name}: out {out.shape} |out|max {np.abs(out).max():.4f}")


if __name__ == "__main__":
    main(sys.argv[1:])
