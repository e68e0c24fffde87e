"""bfi_smp_sample_rows_noalloc (the library's fixed per-device workspace, no allocation)
against bfi_smp_sample_rows (the context's allocated workspace), through the C ABI: the
same tokens on two calls in a row, the second with a smaller input, and the size limit."""
import numpy as np
import pytest

import bfi_smp
import workloads

pytestmark = pytest.mark.gpu


def _sub(cfg, B, V):
    """The first B rows and V logits of a workload (histories folded into [0, V))."""
    sub = dict(cfg)
    sub.update(B=B, V=V, logits=np.ascontiguousarray(cfg["logits"][:B, :V]), params=cfg["params"][:B],
               u=cfg["u"][:B])
    h = [cfg["hist"][cfg["hist_off"][b]:cfg["hist_off"][b + 1]] % V for b in range(B)]
    sub["hist"] = np.concatenate(h).astype(np.uint32)
    sub["hist_off"] = cfg["hist_off"][:B + 1].copy()
    if cfg["mask"] is not None:
        W = (V + 31) // 32
        sub["mask"] = np.ascontiguousarray(cfg["mask"][:B, :W])
    return sub


def _both(smp, cfg):
    import torch

    d = workloads.to_device(cfg)
    ref = torch.full_like(d["out"], -1)
    got = torch.full_like(d["out"], -2)
    smp.sample_rows(d["logits"], d["params"], d["u"], ref, d["hist"], d["hist_off"], d["mask"])
    smp.sample_rows_noalloc(d["logits"], d["params"], d["u"], got, d["hist"], d["hist_off"], d["mask"])
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


def test_noalloc_matches_the_allocating_entry_point(gpu):
    smp = bfi_smp.Sampler(0)
    try:
        # first call: 8 rows of C2 at the full vocabulary; second: 3 rows of a masked
        # workload at a smaller vocabulary (the array keeps the first call's contents)
        for cfg in (_sub(workloads.config("C2", seed=3), 8, 151936),
                    _sub(workloads.config("C3", seed=4), 3, 40000)):
            print(f"[noalloc] B={cfg['B']} V={cfg['V']} mask={cfg['mask'] is not None}", flush=True)
            ref, got = _both(smp, cfg)
            assert np.array_equal(ref, got), (ref, got)
    finally:
        smp.close()


def test_noalloc_rejects_rows_beyond_its_workspace(gpu):
    import torch

    smp = bfi_smp.Sampler(0)
    try:
        cfg = _sub(workloads.config("C2", seed=5), 64, 151936)  # about 64 x 6 MB: too large
        d = workloads.to_device(cfg)
        with pytest.raises(bfi_smp.SamplerError, match="BFI_SMP_NOALLOC_BYTES"):
            smp.sample_rows_noalloc(d["logits"], d["params"], d["u"], d["out"], d["hist"], d["hist_off"],
                                    d["mask"])
        torch.cuda.synchronize()
        # and the entry point still works afterwards
        cfg = _sub(workloads.config("C2", seed=6), 2, 5000)
        ref, got = _both(smp, cfg)
        assert np.array_equal(ref, got), (ref, got)
    finally:
        smp.close()
