"""Oracle (test infrastructure only): the recall worker's bounded exact-MIPS archive.

Restates HeadArchive and ArchiveIndex of src/lazy_recall/recall/cpu_worker.py:17-134 in plain
Python/numpy, with faiss IndexIDMap2(IndexFlatIP) replaced by what it computes: a list of
(position, f32 key) in the order rows were added (removal keeps the others' order), searched by
brute force for the largest inner products (computed in f64), equal products in list order.
"""

from __future__ import annotations

import numpy as np


def bf16_to_float32(values):
    """cpu_worker.py:13-14."""
    return (values.astype(np.uint32) << 16).view(np.float32)


class HeadArchive:
    """cpu_worker.py:17-92."""

    def __init__(self, dimension, capacity):
        self.dimension, self.capacity = dimension, capacity
        self.flat = []  # the index: [position, f32 key] in insertion order
        self.payload = {}
        self.positions = {}  # slot -> position
        self.lookup = {}
        self.free = []
        self.used = 0
        self.cursor = 0
        self.dropped = 0

    def _remove_ids(self, ids):
        ids = set(int(i) for i in ids)
        self.flat = [entry for entry in self.flat if entry[0] not in ids]

    def remove(self, positions):
        selected = [int(p) for p in positions if int(p) in self.lookup]
        if not selected:
            return
        self._remove_ids(selected)
        for position in selected:
            slot = self.lookup.pop(position)
            self.positions[slot] = -1
            self.free.append(slot)

    def add(self, positions, payload):
        if len(np.unique(positions)) != len(positions):
            raise ValueError("Duplicate identities in one archive batch")
        self.remove(positions)
        slots, kept = [], []
        for row, position in enumerate(positions):
            if self.free:
                slot = self.free.pop()
            elif self.used < self.capacity:
                slot = self.used
                self.used += 1
            else:
                slot = self.cursor
                self.cursor = (self.cursor + 1) % self.capacity
                previous = int(self.positions.get(slot, -1))
                if previous >= 0:
                    self._remove_ids([previous])
                    self.lookup.pop(previous)
                    self.dropped += 1
                if slot in slots:
                    earlier = slots.index(slot)
                    slots.pop(earlier)
                    kept.pop(earlier)
            self.payload[slot] = payload[row].copy()
            self.positions[slot] = int(position)
            self.lookup[int(position)] = slot
            slots.append(slot)
            kept.append(row)
        for row in kept:
            self.flat.append([int(positions[row]), bf16_to_float32(payload[row, 0])])

    def search(self, query, topk):
        if not self.lookup:
            return np.empty(0, np.int64), np.empty((0, 2, self.dimension), np.uint16)
        q = np.asarray(query, dtype=np.float64).reshape(-1)
        scores = [float(np.dot(key.astype(np.float64), q)) for _, key in self.flat]
        order = sorted(range(len(self.flat)), key=lambda i: -scores[i])  # stable: list order
        chosen = [self.flat[i][0] for i in order[:min(topk, len(self.lookup))]]
        positions = np.asarray(chosen, dtype=np.int64)
        return positions, np.stack([self.payload[self.lookup[p]] for p in chosen])


class ArchiveIndex:
    """cpu_worker.py:94-134."""

    def __init__(self, layers, heads, dimension, capacity):
        self.layers, self.heads, self.dimension = layers, heads, dimension
        self.indices = [HeadArchive(dimension, capacity) for _ in range(layers * heads)]

    @property
    def size(self):
        return sum(len(index.lookup) for index in self.indices)

    @property
    def dropped(self):
        return sum(index.dropped for index in self.indices)

    def add(self, metadata, payload):
        if metadata.shape != (len(payload), 3) or payload.shape[1:] != (2, self.dimension):
            raise ValueError("Archive payload shape mismatch")
        if (metadata < 0).any() or (metadata[:, 0] >= self.layers).any() or (metadata[:, 1] >= self.heads).any():
            raise ValueError("Invalid archive identity")
        segments = metadata[:, 0] * self.heads + metadata[:, 1]
        for segment in np.unique(segments):
            selected = segments == segment
            self.indices[int(segment)].add(metadata[selected, 2], payload[selected])

    def remove(self, metadata):
        metadata = np.asarray(metadata, dtype=np.int64).reshape(-1, 3)
        segments = metadata[:, 0] * self.heads + metadata[:, 1]
        for segment in np.unique(segments):
            self.indices[int(segment)].remove(metadata[segments == segment, 2])

    def search(self, queries, topk):
        metadata, payload = [], []
        for segment, index in enumerate(self.indices):
            positions, vectors = index.search(queries.reshape(-1, self.dimension)[segment], topk)
            for position, vector in zip(positions, vectors):
                metadata.append((segment // self.heads, segment % self.heads, int(position)))
                payload.append(vector)
        return (np.asarray(metadata, dtype=np.int64).reshape(-1, 3),
                np.asarray(payload, dtype=np.uint16).reshape(-1, 2, self.dimension))
