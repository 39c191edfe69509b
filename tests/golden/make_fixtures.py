"""Write the golden vectors under tests/golden/ from the reference's own functions.

Runs only in the build container, where the reference (TahirSher/KV-Project) is readable:

    python tests/golden/make_fixtures.py [--reference /root/reference]

It imports STRATA_KV.py and QUASAR_KV.py with KV_PROJECT_ROOT / KV_STRATA_OUTPUT_DIR pointed at a
temporary directory (their Config() creates output folders under the project root) and writes,
for the functions whose exact floats or draws nothing but the reference itself fixes:

  strata_codec.npz     uniform_step(b) for b = 1..8 (step, mse; STRATA_KV.py:1132-1155);
                       rotation signs of rotation_matrix(d, "strata") for d = 64, 128 (1110-1128);
                       one side's compression as compress_layer does it (1546-1548): seeded fp32
                       rows X (Hkv, n, d), mu = as_stored(X.mean(1)), Y = (X - mu) @ R.T, and
                       strata_quantize(Y, b) codes and scales for b = 2, 4, 8 (1158-1168)
  quasar_codebooks.npz lloyd_max_gaussian(b), b = 1..4 (STRATA_KV.py:1082-1098); stage_codebooks
                       for (2, 2, 4), (4, 4), (8,) (QUASAR_KV.py:1143-1169) and
                       embedded_quantize codes of seeded coefficients (1172-1183)
  coverage_groups.npz  coverage_groups(H, cfg) (STRATA_KV.py:1206-1222) for several H under the
                       default Config and the reference's test config (1964)
  quasar_state.npz     one seeded fp32 layer (Hq 8, Hkv 2, d 128, H 700; keep 0.5: 458 coded
                       tokens over 23 levels, rank 128) compressed by the
                       reference's own QuasarMethod.compress_layer (QUASAR_KV.py:1628-1710) under
                       its default Config, its stored code QuasarMethod.pack (1786-1808: every step's
                       side / band / stage / n and packed code bytes, rho, T, mu at fp16, the level
                       histogram), the exact rows of native_state (1830-1843), and the output of
                       QuasarState.attend (1952-1977, the reference's PyTorch path) for one query
                       token after one appended token
  strata_state.npz     the layer of layer_inputs.strata_layer (seeded; Hq 8, Hkv 2, d 128, H 700)
                       compressed by the reference's own StrataMethod.compress_layer
                       (STRATA_KV.py:1528-1581) at keep 0.25 under its default Config: the
                       allocation (order, level histogram, bits, distortion ratio), its stored code
                       StrataMethod.pack (1611-1627: per stratum planar codes and fp16 scales, fp16
                       means) and the output of StrataState.attend (1762-1795, the reference's
                       PyTorch path) after one appended token (native_state, 1673-1687)
  kivi_attention.npz   on the seeded inputs of layer_inputs.kivi_inputs: kivi_quant (826-856) codes,
                       fp16 zero points and scales of keys (per channel, groups 32 / 64, 2 and 4 bits,
                       0 and 4 sink rows) and values (per token, groups 32 / 64 / 128); chunked_attention (641-675) over exact
                       entries (causal positions, a per-head hide_at) and token entries (a -inf
                       padding bias, tau) in chunks of 2; snapkv_scores (932-954) under the default
                       Config; tier_reference (1751-1760) of one stratum at 2, 4 and 8 bits

The tests load these files; nothing on the GPU box reads the reference.
"""
from __future__ import annotations

import argparse
import importlib.util
import os
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))


def _load(ref: Path, name: str):
    spec = importlib.util.spec_from_file_location(name, ref / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def strata_codec(S) -> dict:
    import torch
    out = {}
    steps = np.array([S.uniform_step(b)[0] for b in range(1, 9)], np.float64)
    mses = np.array([S.uniform_step(b)[1] for b in range(1, 9)], np.float64)
    out["uniform_step"], out["uniform_mse"] = steps, mses
    for d in (64, 128):
        R = S.rotation_matrix(d, "strata").double().numpy()
        out[f"signs_{d}"] = np.round(R[0] * np.sqrt(d)).astype(np.int8)    # row 0 of H_d is all ones
    rng = np.random.default_rng(20260101)
    Hkv, n, d = 2, 96, 128
    mag = np.abs(rng.standard_t(3, size=(Hkv, 1, d))) + 0.1            # heavy-tailed channel scales
    X = (rng.standard_normal((Hkv, n, d)) * mag + rng.standard_normal((Hkv, 1, d))).astype(np.float32)
    X[0, 5] = X[0, 5].mean()                                           # a row equal to its mean: tiny rms
    X[1, 7] *= 40.0                                                    # one large row
    Xt = torch.from_numpy(X)
    R = S.rotation_matrix(d, "strata")
    mu = S.as_stored(Xt.mean(1, keepdim=True))
    Y = (Xt - mu) @ R.T
    out["X"], out["mu"], out["Y"] = X, mu.numpy().astype(np.float32), Y.numpy().astype(np.float32)
    for b in (2, 4, 8):
        c, s, _ = S.strata_quantize(Y, b)
        out[f"codes_{b}"], out[f"scales_{b}"] = c.numpy(), s.numpy().astype(np.float32)
    return out


def quasar_codebooks(S, Q) -> dict:
    import torch
    out = {}
    for b in range(1, 5):
        out[f"lloyd_{b}"] = S.lloyd_max_gaussian(b).numpy()
    rng = np.random.default_rng(20260102)
    u = torch.from_numpy(rng.standard_normal((2, 64, 16)).astype(np.float32))
    out["u"] = u.numpy()
    for stages in ((2, 2, 4), (4, 4), (8,)):
        tag = "_".join(map(str, stages))
        for t, cb in enumerate(Q.stage_codebooks(stages)):
            out[f"levels_{tag}_{t}"] = cb.numpy()
        codes, _ = Q.embedded_quantize(u, stages)
        for t, c in enumerate(codes):
            out[f"codes_{tag}_{t}"] = c.numpy()
    return out


def quasar_state(Q) -> dict:
    import types
    import torch
    rng = np.random.default_rng(20260103)
    Hq, Hkv, d, H, hidden = 8, 2, 128, 700, 256
    cfg = Q.Config()
    q = rng.standard_normal((1, Hq, H, d)).astype(np.float32) * 1.5
    k = rng.standard_normal((1, Hkv, H, d)).astype(np.float32) * (np.abs(rng.standard_t(3, (1, Hkv, 1, d))) + 0.3)
    v = rng.standard_normal((1, Hkv, H, d)).astype(np.float32)
    k[:, :, 0] += 2.0 * q[0, ::Hq // Hkv].mean(1)[None]                 # a sink the queries lean on
    hot = rng.permutation(H - 64)[:16] + 16                             # a few heavily read tokens
    k[:, :, hot] += 1.5 * q[0, ::Hq // Hkv, -32:].mean(1)[None, :, None]
    Wo = (rng.standard_normal((hidden, Hq * d)) / np.sqrt(Hq * d)).astype(np.float32)
    runner = types.SimpleNamespace(d=d, Hq=Hq, layers=[types.SimpleNamespace(
        self_attn=types.SimpleNamespace(o_proj=types.SimpleNamespace(weight=torch.from_numpy(Wo))))])
    qm = Q.QuasarMethod(cfg, 0.5, "quasar", runner)
    qt, kt, vt = torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v)
    al = qm.compress_layer(0, qt, kt, vt, d ** -0.5, H)
    al["packed"] = qm.pack(al)
    al.pop("sides")
    qm.alloc[0] = al
    st = qm.native_state(0, kt, vt, 2, torch.float32)
    p = st.p
    kn = torch.from_numpy(rng.standard_normal((1, Hkv, 1, d)).astype(np.float32))
    vn = torch.from_numpy(rng.standard_normal((1, Hkv, 1, d)).astype(np.float32))
    qn = torch.from_numpy((rng.standard_normal((1, Hq, 1, d)) * 1.5).astype(np.float32))
    st.append(kn, vn, torch.tensor([H]))
    out = st.attend(qn, d ** -0.5, torch.tensor([H]))
    res = {"stages": np.array(qm.stages, np.int64), "H": np.array(H, np.int64), "n_c": np.array(p["n_c"], np.int64),
           "counts": p["counts"].numpy(), "Ke": st.K[:, :, :st.n0].numpy(), "Ve": st.V[:, :, :st.n0].numpy(),
           "kn": kn.numpy(), "vn": vn.numpy(), "qn": qn.numpy(), "out": out.numpy(),
           "step_meta": np.array([[x["side"], x["a"], x["b"], x["stage"], x["n"]] for x in p["steps"]], np.int64)}
    for i, x in enumerate(p["steps"]):
        res[f"codes_{i}"] = x["codes"].numpy()
    for nm in ("rho_k", "rho_v", "T_k", "T_v", "mu_k", "mu_v"):
        res[nm] = p[nm].to(torch.float16).numpy()
    return res


def strata_state(S) -> dict:
    import types
    import torch
    from layer_inputs import strata_layer
    q, k, v, Wo, kn, vn, qn = strata_layer()
    Hq, Hkv, H, d = q.shape[1], k.shape[1], k.shape[2], k.shape[3]
    runner = types.SimpleNamespace(d=d, Hq=Hq, layers=[types.SimpleNamespace(
        self_attn=types.SimpleNamespace(o_proj=types.SimpleNamespace(weight=torch.from_numpy(Wo))))])
    sm = S.StrataMethod(S.Config(), 0.25, "strata", runner)
    kt, vt = torch.from_numpy(k), torch.from_numpy(v)
    al = sm.compress_layer(0, torch.from_numpy(q), kt, vt, d ** -0.5, H)
    al["packed"] = sm.pack(al)
    sm.alloc[0] = al
    st = sm.native_state(0, kt, vt, 2, torch.float32)
    st.append(torch.from_numpy(kn), torch.from_numpy(vn), torch.tensor([H]))
    out = st.attend(torch.from_numpy(qn), d ** -0.5, torch.tensor([H]))
    p = al["packed"]
    res = {"keep": np.array(0.25), "counts": np.array(al["counts"], np.int64), "n_ex": np.array(al["n_ex"], np.int64),
           "n_c": np.array(al["n_c"], np.int64), "bits": np.array(al["bits"], np.float64),
           "distortion": np.array(al["distortion"], np.float64), "order": al["order"].numpy().astype(np.int16),
           "rs": np.array(al["rs"], np.int64), "re": np.array(al["re"], np.int64), "n0": np.array(st.n0, np.int64),
           "tier_meta": np.array([[t["bits"], t["n"]] for t in p["tiers"]], np.int64), "out": out.numpy(),
           "payload": np.array(sm.payload(0), np.int64)}
    for i, t in enumerate(p["tiers"]):
        for x in ("kc", "vc", "ks", "vs"):
            res[f"{x}_{i}"] = t[x].numpy()
    if al["n_c"]:
        res["mu_k"], res["mu_v"] = p["mu_k"].numpy(), p["mu_v"].numpy()
    return res


def kivi_attention(S) -> dict:
    import torch
    from layer_inputs import kivi_inputs
    x = kivi_inputs()
    t = {k: torch.from_numpy(v) for k, v in x.items() if isinstance(v, np.ndarray)}
    out = {}
    for bits in (2, 4):
        for group in (32, 64):
            for sink in (0, 4):
                r = S.kivi_quant(t["K"], bits, group, True, sink)
                tag = f"k_{bits}_{group}_{sink}"
                out[f"{tag}_codes"] = r["codes"].numpy()
                out[f"{tag}_lo"], out[f"{tag}_scale"] = r["lo"].numpy(), r["scale"].numpy()
        for group in (32, 64, 128):
            r = S.kivi_quant(t["V"], bits, group, False, 0)
            tag = f"v_{bits}_{group}"
            out[f"{tag}_codes"] = r["codes"].numpy()
            out[f"{tag}_lo"], out[f"{tag}_scale"] = r["lo"].numpy(), r["scale"].numpy()
    q_pos = torch.tensor([97, 98, 99])
    kv_pos = torch.arange(100)
    hide = torch.full((1, 2, 100), 10 ** 9, dtype=torch.long)
    hide[0, 0, 10:20] = 98                       # head 0: ten entries hidden from position 98 on
    b = torch.zeros((1, 2, 50))
    b[:, :, 45:] = float("-inf")                 # padding entries
    tok = {"k": t["tk"], "v": t["tv"], "b": b, "tau": torch.arange(50) + 60}
    out["attn"] = S.chunked_attention(t["qa"], 128 ** -0.5, q_pos, t["K"], t["V"], kv_pos, hide, tok, 2).numpy()
    cfg = S.Config()
    out["snap_params"] = np.array([cfg.SNAPKV_WINDOW, cfg.SNAPKV_KERNEL], np.int64)
    out["snap"] = S.snapkv_scores(t["qs"], t["ks"], 300, 128 ** -0.5, cfg).numpy()
    for bits in (2, 4, 8):
        ck, cv = x["codes"][bits]
        sk, sv = x["scales"][bits]
        tier = {"bits": bits, "kc": S.pack_planar(torch.from_numpy(ck), bits), "vc": S.pack_planar(torch.from_numpy(cv), bits),
                "ks": torch.from_numpy(sk).to(torch.float16), "vs": torch.from_numpy(sv).to(torch.float16)}
        m, l_, acc, z = S.StrataState.tier_reference(t["qr"], t["qb"], tier)
        out[f"tier_{bits}_m"], out[f"tier_{bits}_l"], out[f"tier_{bits}_acc"] = m.numpy(), l_.numpy(), acc.numpy()
    return out


def coverage_groups(S) -> dict:
    from dataclasses import replace
    out = {}
    cfgs = {"default": S.Config(), "test": replace(S.Config(), STRATA_SEGMENT=64, STRATA_QUERIES=8, STRATA_LOCAL=16)}
    for name, cfg in cfgs.items():
        out[f"{name}_params"] = np.array([cfg.N_SINK, cfg.STRATA_LOCAL, cfg.W_OBS, cfg.STRATA_SEGMENT,
                                          cfg.STRATA_QUERIES], np.int64)
        for H in (200, 700, 1500, 4100):
            groups = S.coverage_groups(H, cfg)
            out[f"{name}_{H}_lengths"] = np.array([len(g) for g in groups], np.int64)
            out[f"{name}_{H}_positions"] = np.concatenate(groups).astype(np.int64)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    a = ap.parse_args()
    ref = Path(a.reference)
    tmp = tempfile.mkdtemp(prefix="kvref_")
    os.environ["KV_PROJECT_ROOT"] = tmp
    os.environ["KV_STRATA_OUTPUT_DIR"] = tmp
    S = _load(ref, "STRATA_KV")
    Q = _load(ref, "QUASAR_KV")
    for name, data in (("strata_codec", strata_codec(S)), ("quasar_codebooks", quasar_codebooks(S, Q)),
                       ("coverage_groups", coverage_groups(S)), ("quasar_state", quasar_state(Q)),
                       ("strata_state", strata_state(S)), ("kivi_attention", kivi_attention(S))):
        np.savez_compressed(HERE / f"{name}.npz", **data)
        print(f"wrote {name}.npz ({(HERE / f'{name}.npz').stat().st_size} bytes, {len(data)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
