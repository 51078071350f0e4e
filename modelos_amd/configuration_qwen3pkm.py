"""Qwen3PKMConfig: the model configuration the reference's modeling code reads.

The reference's configuration_qwen3pkm.py (configuration_qwen3pkm.py:4-109)
does not parse (an unterminated string at :99), so the modeling file cannot
import it. This is a valid class with the same name, base class (transformers'
Qwen3Config), model_type, field names and defaults, and the checks the
reference means to make: only "hidden" query / value sources, and PKM /
fast-weight layer indices inside the stack.
"""
from __future__ import annotations

from transformers.models.qwen3.configuration_qwen3 import Qwen3Config

# field -> default, in the reference's order (configuration_qwen3pkm.py:9-51)
PKM_DEFAULTS = {
    "pkm_layers": None,
    "pkm_k_dim": 512,
    "pkm_v_dim": 512,
    "pkm_heads": 4,
    "pkm_topk": 32,
    "pkm_n_subkeys": 512,
    "pkm_query_rmsnorm": True,
}
FWPKM_DEFAULTS = {
    "fwpkm_layers": None,
    "fwpkm_k_dim": 512,
    "fwpkm_v_dim": 512,
    "fwpkm_heads": 1,
    "fwpkm_topk": 8,
    "fwpkm_n_subkeys": 512,
    "fwpkm_variant": "pkm",  # "pkm" | "mlp"
    "fwpkm_fp32_fw": True,
    "fwpkm_before_attn": True,
    "fwpkm_update_chunk_size": 512,
    "fwpkm_loss_type": "mse",
    "fwpkm_optimizer_type": "sgd",
    "fwpkm_optimizer_lr": 1.0,
    "fwpkm_optimizer_weight_decay": 0.0,
    "fwpkm_grad_clip": False,
    "fwpkm_addr_loss": "me",  # None | "me"
    "fwpkm_addr_loss_weight": 1.0,
    "fwpkm_weight_loss_with_gates": True,
    "fwpkm_mem_grad_to_values_only": True,
    "fwpkm_query_src": "hidden",
    "fwpkm_value_src": "hidden",
    "fwpkm_compress_query": None,  # None | "l2norm" | "zero_mean"
    "fwpkm_compress_value": "zero_mean",  # None | "l2norm" | "zero_mean"
    "fwpkm_target_value_lookahead": 1,
    "fwpkm_score_nonlinear": "softmax",  # "softmax" | "silu" | "relu"
    "fwpkm_qk_score_type": "idw",  # "dot_product" | "idw"
    "fwpkm_score_temperature": 1.0,
    "fwpkm_out_fuse_gate": True,
}


class Qwen3PKMConfig(Qwen3Config):
    """Qwen3 configuration plus the product-key memory (pkm_*, replacing the
    MLP of the layers in pkm_layers) and fast-weight memory (fwpkm_*, an extra
    block in the layers in fwpkm_layers) fields."""

    model_type = "qwen3_pkm"

    def __init__(
        self,
        pkm_layers=None,
        pkm_k_dim=512,
        pkm_v_dim=512,
        pkm_heads=4,
        pkm_topk=32,
        pkm_n_subkeys=512,
        pkm_query_rmsnorm=True,
        fwpkm_layers=None,
        fwpkm_k_dim=512,
        fwpkm_v_dim=512,
        fwpkm_heads=1,
        fwpkm_topk=8,
        fwpkm_n_subkeys=512,
        fwpkm_variant="pkm",
        fwpkm_fp32_fw=True,
        fwpkm_before_attn=True,
        fwpkm_update_chunk_size=512,
        fwpkm_loss_type="mse",
        fwpkm_optimizer_type="sgd",
        fwpkm_optimizer_lr=1.0,
        fwpkm_optimizer_weight_decay=0.0,
        fwpkm_grad_clip=False,
        fwpkm_addr_loss="me",
        fwpkm_addr_loss_weight=1.0,
        fwpkm_weight_loss_with_gates=True,
        fwpkm_mem_grad_to_values_only=True,
        fwpkm_query_src="hidden",
        fwpkm_value_src="hidden",
        fwpkm_compress_query=None,
        fwpkm_compress_value="zero_mean",
        fwpkm_target_value_lookahead=1,
        fwpkm_score_nonlinear="softmax",
        fwpkm_qk_score_type="idw",
        fwpkm_score_temperature=1.0,
        fwpkm_out_fuse_gate=True,
        **kwargs,
    ):
        super().__init__(**kwargs)
        fields = dict(locals())
        for name in (*PKM_DEFAULTS, *FWPKM_DEFAULTS):
            setattr(self, name, fields[name])
        self.pkm_layers = list(pkm_layers) if pkm_layers is not None else []
        self.fwpkm_layers = list(fwpkm_layers) if fwpkm_layers is not None else []
        self.num_fwpkm_layers = len(self.fwpkm_layers)
        if self.fwpkm_query_src != "hidden" or self.fwpkm_value_src != "hidden":
            raise NotImplementedError(
                "Qwen3PKMConfig supports only fwpkm_query_src='hidden' and fwpkm_value_src='hidden'"
            )
        for kind, layers in (("pkm_layers", self.pkm_layers), ("fwpkm_layers", self.fwpkm_layers)):
            for layer in layers:
                if not 0 <= layer < self.num_hidden_layers:
                    raise ValueError(f"{kind} contains invalid layer index {layer}")


__all__ = ["Qwen3PKMConfig"]
