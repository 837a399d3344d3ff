"""Write golden route-table vectors from the reference's own route builder.

Run only in the build container, where the read-only reference checkout is
mounted (default ``/root/reference``, override with ``TRMOE_REFERENCE``)::

    python tests/golden/make_reference_vectors.py

Why an import is needed: the exact salts, strides and permutations of the
route strategies (``complexity/tr_hash/routing.py:12-259``) and the pair code
layout (``routing.py:262-311``) are not fixed by any invariant the
reference's tests state (balance, distinctness and layer dependence would
all survive a swapped constant).  So those two functions are pinned by their
own outputs.  Nothing else is imported, and the GPU box never runs this file:
it only reads the fixtures written here.

Outputs (``tests/golden/``):

* ``route_tables_v32000.npz`` -- full multi-hash tables, V=32000, top-2,
  layer 0, E in {4, 8, 16}, as uint8;
* ``route_digests.json`` -- SHA-256 of the int64 table bytes for every
  (strategy, E, k, layer, V, hash_count) case the tests check, plus the first
  32 columns of each table in clear;
* ``pair_codes_v997.npz`` -- ``compile_top2_pair_metadata`` outputs.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = os.environ.get("TRMOE_REFERENCE", "/root/reference")

MULTI_V32000 = [(4, layer) for layer in range(16)] + [(8, 0), (16, 0)]
SMALL_STRATEGIES = [
    "modulo_cyclic",
    "token_id_balanced_hash",
    "token_id_affine_hash",
    "token_id_multi_hash",
]
SMALL_SHAPES = [(2, 1), (4, 2), (8, 4), (16, 4), (8, 2), (16, 2)]


def _digest(table: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(table, dtype=np.int64).tobytes()).hexdigest()


def main() -> None:
    sys.path.insert(0, REF)
    from complexity.tr_hash import TRHashEngineConfig  # noqa: E402
    from complexity.tr_hash.routing import (  # noqa: E402
        build_route_table,
        compile_top2_pair_metadata,
    )

    cases = []
    full = {}

    def record(strategy, vocab, experts, top_k, layer, hash_count=2, keep=False):
        config = TRHashEngineConfig(
            hidden_size=8,
            vocab_size=vocab,
            num_experts=experts,
            top_k=top_k,
            expert_width=4,
            routing_strategy=strategy,
            layer_index=layer,
            route_hash_count=hash_count,
        )
        table = build_route_table(config).numpy().astype(np.int64)
        cases.append(
            dict(
                strategy=strategy,
                vocab_size=vocab,
                num_experts=experts,
                top_k=top_k,
                layer_index=layer,
                hash_count=hash_count,
                sha256=_digest(table),
                head=table[:, :32].tolist(),
            )
        )
        if keep:
            full[f"multi_e{experts}_l{layer}"] = table.astype(np.uint8)
        return table

    for experts, layer in MULTI_V32000:
        record("token_id_multi_hash", 32000, experts, 2, layer, keep=(layer == 0))
    for strategy in SMALL_STRATEGIES:
        for experts, top_k in SMALL_SHAPES:
            record(strategy, 997, experts, top_k, 3)
    for experts, top_k in [(4, 2), (8, 2), (8, 4), (16, 4)]:
        record("token_id_hierarchical_hash", 997, experts, top_k, 3)
    for hash_count in (3, 8):
        record("token_id_multi_hash", 4093, 4, 2, 0, hash_count=hash_count)
    record("token_id_multi_hash", 4093, 4, 2, 1)

    pair = {}
    for strategy in SMALL_STRATEGIES:
        for experts in (2, 4, 8):
            config = TRHashEngineConfig(
                hidden_size=8,
                vocab_size=997,
                num_experts=experts,
                top_k=2,
                expert_width=4,
                routing_strategy=strategy,
                layer_index=3,
            )
            routes = build_route_table(config)
            codes, pairs = compile_top2_pair_metadata(routes, num_experts=experts)
            pair[f"{strategy}_e{experts}_codes"] = codes.numpy()
            pair[f"{strategy}_e{experts}_pairs"] = pairs.numpy()
            pair[f"{strategy}_e{experts}_routes"] = routes.numpy().astype(np.uint8)

    np.savez_compressed(HERE / "route_tables_v32000.npz", **full)
    np.savez_compressed(HERE / "pair_codes_v997.npz", **pair)
    with open(HERE / "route_digests.json", "w") as handle:
        json.dump({"route_seed": 0x71D5A17, "cases": cases}, handle, indent=1)
    print(f"wrote {len(cases)} digests, {len(full)} full tables, {len(pair) // 3} pair sets")


if __name__ == "__main__":
    main()
