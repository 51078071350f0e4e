"""Writes golden vectors of the reference's HashingMemory (pkm/memory.py) on the CPU.

Run in a checkout that has the reference at REFERENCE (default
/root/reference):  python tests/golden/make_pkm_layer_golden.py [case ...]
(all cases when none is named)

The reference module is imported only here, on the CPU, to pin the one
thing no closed form covers: the composition of its forward (query network,
norm, get_indices layout, softmax, embedding bag, swilu projection) and the
gradients autograd takes through it. Every parameter, the input and the
upstream gradient are stored explicitly (no reliance on construction RNG
order), float32, with inputs drawn so the top-k selections are tie-free.

Output: tests/golden/pkm_layer_<case>.pt — a dict of tensors, loadable with
torch.load(weights_only=True). The value table's gradient is stored as the
rows it touches ("grad_rows.<name>") and their values ("grad.<name>").
"""
from __future__ import annotations

import hashlib
import os
import sys
from pathlib import Path

import torch

REFERENCE = os.environ.get("REFERENCE", "/root/reference")
OUT = Path(__file__).resolve().parent

CASES = {
    # RMSNorm query (the layer's default), swilu projection
    "rmsnorm": dict(input_dim=64, output_dim=32, mem_k_dim=64, mem_heads=2, mem_knn=8, mem_n_keys=64,
                    mem_query_rmsnorm=True, mem_query_batchnorm=False),
    # BatchNorm query in train mode, 4 heads (the CPU parity configuration's choices, smaller)
    "batchnorm": dict(input_dim=48, output_dim=32, mem_k_dim=128, mem_heads=4, mem_knn=16, mem_n_keys=64,
                      mem_query_rmsnorm=False, mem_query_batchnorm=True),
    # a value width different from the output width (the model's pkm_v_dim 512 vs hidden 1024, smaller)
    "vdim": dict(input_dim=64, output_dim=32, mem_k_dim=64, mem_heads=2, mem_knn=8, mem_n_keys=64, mem_v_dim=16,
                 mem_query_rmsnorm=True, mem_query_batchnorm=False),
}
BATCH, SEQ = 2, 12


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def main():
    sys.path.insert(0, REFERENCE)
    from pkm.memory import HashingMemory  # noqa: E402  (reference, CPU only)

    names = sys.argv[1:] or list(CASES)
    for name in names:
        kw = CASES[name]
        torch.manual_seed(0)
        mem = HashingMemory(**kw)
        g = torch.Generator().manual_seed(1234)
        params = {}
        for pname, p in mem.named_parameters():
            if pname == "keys":
                v = (torch.rand(p.shape, generator=g) * 2 - 1) / 16  # U(-1/16, 1/16)
            elif pname.endswith("values.weight"):
                v = torch.randn(p.shape, generator=g) * p.shape[1] ** -0.5
            elif pname.endswith("norm.weight"):
                v = 1 + 0.1 * torch.randn(p.shape, generator=g)
            else:
                v = torch.randn(p.shape, generator=g) * 0.1
            with torch.no_grad():
                p.copy_(v)
            params[pname] = v.clone()
        mem.train()
        x = torch.randn((BATCH, SEQ, kw["input_dim"]), generator=g).requires_grad_(True)
        dout = torch.randn((BATCH, SEQ, kw["output_dim"]), generator=g)
        out, idx = mem(x)
        out.backward(dout)
        rec = {
            "x": x.detach().clone(),
            "dout": dout,
            "out": out.detach().clone(),
            "indices": idx.clone(),
            "dx": x.grad.clone(),
        }
        for pname, v in params.items():
            rec["param." + pname] = v
        for pname, p in mem.named_parameters():
            if pname.endswith("values.weight"):
                # the value table's gradient is zero outside the looked-up rows: store those rows only
                rows = (p.grad.abs().sum(1) != 0).nonzero().squeeze(1)
                rec["grad_rows." + pname] = rows
                rec["grad." + pname] = p.grad[rows].clone()
            else:
                rec["grad." + pname] = p.grad.clone()
        rec["sha256.x"] = torch.tensor(list(bytes.fromhex(sha(rec["x"]))), dtype=torch.uint8)
        rec["config"] = torch.tensor([kw["input_dim"], kw["output_dim"], kw["mem_k_dim"], kw["mem_heads"],
                                      kw["mem_knn"], kw["mem_n_keys"], int(kw["mem_query_batchnorm"]),
                                      kw.get("mem_v_dim", -1)])
        path = OUT / f"pkm_layer_{name}.pt"
        torch.save(rec, path)
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
