"""Sizes the HIP kernels have no path for raise a clear error when the
module is built, not a kernel status code mid-forward (CPU only: nothing
runs on the device)."""
import pytest

from modelos_amd.pkm.memory import HashingMemory
from modelos_amd.product_keys import check_supported


@pytest.mark.parametrize("kw,needle", [
    (dict(mem_n_keys=20000), "n_keys=20000"),
    (dict(mem_knn=2000, mem_n_keys=4096), "knn=2000"),
    (dict(mem_knn=80), "knn=80 > n_keys=64"),
    (dict(output_dim=48), "value dim=48"),
    (dict(mem_v_dim=24), "value dim=24"),
])
def test_unsupported_layer_sizes_raise_at_construction(kw, needle):
    args = dict(input_dim=64, output_dim=64, mem_k_dim=64, mem_heads=2, mem_knn=8, mem_n_keys=64)
    args.update(kw)
    with pytest.raises(NotImplementedError, match=needle):
        HashingMemory(**args)


def test_supported_sizes_pass():
    for n_keys, k_dim, knn, v in [(64, 32, 1, 4), (1024, 512, 32, 1024), (2048, 512, 64, 2048), (512, 256, 16, 4096),
                                  (100, 20, 80, 64), (4096, 512, 128, 1024), (1000, 510, 1000, 8), (16384, 2, 1024, 4)]:
        check_supported(n_keys, k_dim, knn, v)


def test_odd_key_dim_raises():
    with pytest.raises(NotImplementedError, match="k_dim=21"):
        check_supported(64, 21, 8)
