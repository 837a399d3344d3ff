"""MI355X-native TR-MoE feed-forward (TRHashEngine / TRHashEngineMLP).

``complexity_amd.tr_hash`` mirrors ``complexity.tr_hash``;
``complexity_amd.core.mlp.tr_hash_engine.TRHashEngineMLP`` mirrors the
reference's MLP plug-in; ``complexity_amd.ops`` exposes the HIP kernels of
``libtrmoe`` (C ABI in include/trmoe.h) on torch tensors.
"""

__version__ = "0.1.0"
