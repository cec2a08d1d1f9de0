"""spbitnet_amd -- MI355X (gfx950) implementation of spbitnet's 2:4
sparse-ternary linear-layer hot path.

* ``include/spbitnet_amd.h``        C ABI of the HIP library (the drop-in boundary)
* ``spbitnet_amd/csrc/*.hip``       hand-written gfx950 kernels behind it
* ``spbitnet_amd.kernels``          the reference's kernel API, in Python, over the C ABI
* ``spbitnet_amd.model``            Model / InferenceEngine: loader, random-init
                                    models and the decode engines over the C ABI
* ``spbitnet_amd.weights``          host-side format: generation and packing
"""
from .weights import (  # noqa: F401
    PackedLayer,
    make_layer_from_latent,
    meta_words_per_row,
    normal_f32,
    pack,
    random_layer,
    seed_for,
    top2_mask,
    unpack,
    values_words_per_row,
)

__all__ = [
    "PackedLayer", "make_layer_from_latent", "meta_words_per_row", "normal_f32", "pack",
    "random_layer", "seed_for", "top2_mask", "unpack", "values_words_per_row",
]
