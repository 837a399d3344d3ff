"""Static graph buckets for TR-Hash inference (behaviour of complexity/tr_hash/buckets.py)."""

from __future__ import annotations

from typing import Iterable, Tuple

from .config import GraphBucket


def _order(bucket: GraphBucket):
    return (bucket.token_capacity, bucket.batch_size, bucket.sequence_length)


class GraphBucketPlanner:
    """Pick the smallest configured bucket that contains a (batch, sequence) shape."""

    def __init__(self, buckets: Iterable[GraphBucket]):
        self.buckets: Tuple[GraphBucket, ...] = tuple(sorted(set(buckets), key=_order))
        if not self.buckets:
            raise ValueError("at least one CUDA Graph bucket is required")

    def select(self, batch_size: int, sequence_length: int) -> GraphBucket:
        if batch_size <= 0 or sequence_length <= 0:
            raise ValueError("input batch and sequence dimensions must be positive")
        for bucket in self.buckets:  # already in ascending capacity order
            if bucket.batch_size >= batch_size and bucket.sequence_length >= sequence_length:
                return bucket
        raise ValueError(
            f"no CUDA Graph bucket can contain input shape ({batch_size}, {sequence_length})"
        )
