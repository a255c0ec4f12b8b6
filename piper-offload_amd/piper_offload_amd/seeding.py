"""Stable seed derivation (P/seeding.py:10-36).

``derive_seed`` hashes a versioned, typed encoding of its parts with
BLAKE2s (8-byte digest) and returns the little-endian uint64.  The encoding
is a format, so it is kept byte-for-byte identical to the reference: a prefix
``b"piper-offload-seed-v1\\0"``, strings as ``b"s"`` + 8-byte LE length +
UTF-8, integers as ``b"i"`` + 8-byte LE value in [0, 2**64).
"""

from hashlib import blake2s

__all__ = ["derive_seed"]

_UINT64_LIMIT = 1 << 64


def derive_seed(*parts: str | int) -> int:
    """Return a stable unsigned 64-bit seed derived from typed identity parts."""
    digest = blake2s(digest_size=8)
    digest.update(b"piper-offload-seed-v1\0")
    for part in parts:
        if isinstance(part, str):
            data = part.encode("utf-8")
            digest.update(b"s" + len(data).to_bytes(8, "little") + data)
        elif isinstance(part, int) and not isinstance(part, bool):
            if not 0 <= part < _UINT64_LIMIT:
                raise ValueError("derive_seed() integer parts must be unsigned 64-bit values")
            digest.update(b"i" + part.to_bytes(8, "little"))
        else:
            raise TypeError("derive_seed() parts must be strings or unsigned 64-bit integers")
    return int.from_bytes(digest.digest(), "little")
