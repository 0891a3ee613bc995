"""Small synthetic packed stores for the CPU tests (random nibbles and
positive fp16 scales; the bytes, not the numbers, matter here)."""
import numpy as np
import torch

from hydranet_amd.cache.blob_layout import BlobLayout


def random_expert(seed: int, H: int, I: int, g: int) -> dict:
    rng = np.random.default_rng(seed)
    out = {}
    for name, (shape, dt) in BlobLayout.shapes(H, I, g).items():
        if dt == "uint8":
            out[name] = torch.from_numpy(rng.integers(0, 256, size=shape, dtype=np.uint8))
        else:
            out[name] = torch.from_numpy((rng.random(shape) * 0.01 + 1e-4).astype(np.float16))
    return out


def make_store(path, num_layers=2, num_experts=4, H=256, I=512, g=128, model_type=None):
    """experts.bin/.idx under path; returns {(layer, expert): tensors}."""
    from hydranet_amd.preprocess.pack_store import write_packed_store
    experts = {(l, e): random_expert(1000 * l + e, H, I, g)
               for l in range(num_layers) for e in range(num_experts)}
    write_packed_store(path, ((l, e, t) for (l, e), t in experts.items()), num_layers,
                       num_experts, H, I, g, model_type)
    return experts
