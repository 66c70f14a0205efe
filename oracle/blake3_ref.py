"""Pure-Python BLAKE3 (default hash mode, 32-byte digest), TEST INFRASTRUCTURE.

Written from the published BLAKE3 specification with the tree in its
recursive form: a subtree over n > 1 chunks splits into a left subtree of the
largest power of two of chunks strictly below n and a right subtree of the
rest. libholo_hip.so folds the tree with the incremental hasher's stack
instead; comparing the two on many lengths checks the fold. Used by the
`.holo` oracle reader (oracle/graph.py) and by tests only.
"""
from __future__ import annotations

import struct

IV = (0x6A09E667, 0xBB67AE85, 0x3C6EF372, 0xA54FF53A,
      0x510E527F, 0x9B05688C, 0x1F83D9AB, 0x5BE0CD19)
PERM = (2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8)
CHUNK_START, CHUNK_END, PARENT, ROOT = 1, 2, 4, 8
CHUNK, BLOCK = 1024, 64
M32 = 0xFFFFFFFF


def _rotr(x, n):
    return ((x >> n) | (x << (32 - n))) & M32


def _g(s, a, b, c, d, x, y):
    s[a] = (s[a] + s[b] + x) & M32
    s[d] = _rotr(s[d] ^ s[a], 16)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 12)
    s[a] = (s[a] + s[b] + y) & M32
    s[d] = _rotr(s[d] ^ s[a], 8)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 7)


def compress(cv, block_words, counter, blen, flags):
    s = list(cv) + list(IV[:4]) + [counter & M32, (counter >> 32) & M32, blen, flags]
    m = list(block_words)
    for r in range(7):
        _g(s, 0, 4, 8, 12, m[0], m[1])
        _g(s, 1, 5, 9, 13, m[2], m[3])
        _g(s, 2, 6, 10, 14, m[4], m[5])
        _g(s, 3, 7, 11, 15, m[6], m[7])
        _g(s, 0, 5, 10, 15, m[8], m[9])
        _g(s, 1, 6, 11, 12, m[10], m[11])
        _g(s, 2, 7, 8, 13, m[12], m[13])
        _g(s, 3, 4, 9, 14, m[14], m[15])
        if r < 6:
            m = [m[i] for i in PERM]
    return [s[i] ^ s[i + 8] for i in range(8)]


def _words(block: bytes):
    return struct.unpack("<16I", block.ljust(BLOCK, b"\0"))


def _chunk_cv(data: bytes, index: int, root: bool):
    cv = list(IV)
    nblocks = max(1, (len(data) + BLOCK - 1) // BLOCK)
    for b in range(nblocks):
        blk = data[b * BLOCK:(b + 1) * BLOCK]
        flags = (CHUNK_START if b == 0 else 0)
        if b == nblocks - 1:
            flags |= CHUNK_END | (ROOT if root else 0)
        cv = compress(cv, _words(blk), index, len(blk), flags)
    return cv


def _subtree(data: bytes, first_chunk: int, root: bool):
    n = max(1, (len(data) + CHUNK - 1) // CHUNK)
    if n == 1:
        return _chunk_cv(data, first_chunk, root)
    left_chunks = 1 << ((n - 1).bit_length() - 1)   # largest power of two < n
    split = left_chunks * CHUNK
    lcv = _subtree(data[:split], first_chunk, False)
    rcv = _subtree(data[split:], first_chunk + left_chunks, False)
    return compress(IV, lcv + rcv, 0, BLOCK, PARENT | (ROOT if root else 0))


def blake3(data: bytes) -> bytes:
    return struct.pack("<8I", *_subtree(bytes(data), 0, True))
