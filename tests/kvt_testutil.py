"""Shared builders of the GPU parity tests: seeded slot pools of every kind (random codes and scales, an owner table
in which about 80 % of the ring rows belong to one slot of their residue class, random smoothing constants) and the
oracle's dequantized rows of given slots (oracle/ref.py dequant4 / dequant8 / dequant_slots_tiered)."""
import torch

from oracle import ref

D = 256


def slot_pools(slots: int, R: int, g8: int, gen: torch.Generator, H: int = 2) -> dict:
    k4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, generator=gen)
    v4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, generator=gen)
    ks4 = (0.05 + 0.3 * torch.rand(slots, H, D // 32, generator=gen)).half()
    vs4 = (0.05 + 0.3 * torch.rand(slots, H, D // 32, generator=gen)).half()
    rk = torch.randint(-127, 128, (R, H, D), dtype=torch.int8, generator=gen)
    rv = torch.randint(-127, 128, (R, H, D), dtype=torch.int8, generator=gen)
    rks = (0.002 + 0.02 * torch.rand(R, H, D // g8, generator=gen)).half()
    rvs = (0.002 + 0.02 * torch.rand(R, H, D // g8, generator=gen)).half()
    k8 = torch.randint(-127, 128, (slots, H, D), dtype=torch.int8, generator=gen)
    v8 = torch.randint(-127, 128, (slots, H, D), dtype=torch.int8, generator=gen)
    ks8 = (0.002 + 0.02 * torch.rand(slots, H, D // g8, generator=gen)).half()
    vs8 = (0.002 + 0.02 * torch.rand(slots, H, D // g8, generator=gen)).half()
    owner = torch.full((R,), -1, dtype=torch.int32)
    pick = torch.rand(R, generator=gen) < 0.8
    cls = torch.randint(0, slots // R, (R,), generator=gen)
    owner[pick] = (torch.arange(R) + R * cls)[pick].to(torch.int32)
    sm_k = (0.5 + torch.rand(H, D, generator=gen)).half()
    sm_v = (0.5 + torch.rand(H, D, generator=gen)).half()
    return dict(k4=k4, v4=v4, ks4=ks4, vs4=vs4, rk=rk, rv=rv, rks=rks, rvs=rvs, k8=k8, v8=v8, ks8=ks8, vs8=vs8,
                owner=owner, sm_k=sm_k, sm_v=sm_v)


def slot_rows(kind: str, p: dict, slots: torch.Tensor, R: int, g8: int):
    """bf16 K, V rows [n, H, D] of the given slots as the gathers write them."""
    if kind == "tiered":
        return ref.dequant_slots_tiered(slots, p["k4"], p["v4"], p["ks4"], p["vs4"], p["rk"], p["rv"], p["rks"],
                                        p["rvs"], p["owner"], R - 1, p["sm_k"], p["sm_v"], group8=g8)
    sl = slots.long()
    if kind == "int4":
        return ref.dequant4(p["k4"][sl], p["ks4"][sl], p["sm_k"]), ref.dequant4(p["v4"][sl], p["vs4"][sl], p["sm_v"])
    return (ref.dequant8(p["k8"][sl], p["ks8"][sl], p["sm_k"], g8),
            ref.dequant8(p["v8"][sl], p["vs8"][sl], p["sm_v"], g8))


def pool_args(kind: str, p: dict, R: int, dev: str) -> dict:
    """Keyword arguments of the operator surface for one pool kind (device copies)."""
    d = {k: v.to(dev) for k, v in p.items()}
    if kind == "tiered":
        return dict(k_buf=d["k4"], v_buf=d["v4"], k_scale=d["ks4"], v_scale=d["vs4"], sm_k=d["sm_k"], sm_v=d["sm_v"],
                    kv_bits=4, ring_k=d["rk"], ring_v=d["rv"], ring_ks=d["rks"], ring_vs=d["rvs"], owner=d["owner"],
                    ring_mask=R - 1)
    if kind == "int4":
        return dict(k_buf=d["k4"], v_buf=d["v4"], k_scale=d["ks4"], v_scale=d["vs4"], sm_k=d["sm_k"], sm_v=d["sm_v"],
                    kv_bits=4)
    return dict(k_buf=d["k8"], v_buf=d["v8"], k_scale=d["ks8"], v_scale=d["vs8"], sm_k=d["sm_k"], sm_v=d["sm_v"],
                kv_bits=8)


def close(got: torch.Tensor, exp: torch.Tensor, max_abs: float = 2e-3, mean_abs: float = 1e-3) -> None:
    """Same NaN pattern, and the finite entries within max_abs / mean_abs of the fp32 oracle."""
    fin = torch.isfinite(exp)
    assert torch.equal(fin, torch.isfinite(got)), "NaN pattern differs from the oracle"
    if fin.any():
        err = (got[fin].float() - exp[fin]).abs()
        assert float(err.max()) <= max_abs and float(err.mean()) <= mean_abs, (float(err.max()), float(err.mean()))
