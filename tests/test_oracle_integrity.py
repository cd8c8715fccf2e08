"""The digest-table oracle against FIPS 180-4 example messages and the reference's recorded vector."""

import numpy as np

from oracle.integrity import digest_table

# FIPS 180-4 / NIST CSRC SHA-256 examples (one block, two blocks) and the empty message.
KNOWN = {
    b"abc": "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad",
    b"": "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855",
    b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq":
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
    b"abcdefghbcdefghicdefghijdefghijkefghijklfghijklmghijklmnhijklmnoijklmnopjklmnopqklmnopqrlmnopqrsmnopqrst"
    b"nopqrstu": "cf5b16a778af8380036ce59e7b0492370b249b11e8f07a51afac45037afee9d1",
}


def test_known_answers():
    for message, digest in KNOWN.items():
        if message:
            assert digest_table(message).tobytes().hex() == digest
    # equal chunks give equal rows
    table = digest_table(b"a" * 3 * 4096)
    assert (table == table[0]).all()


def test_chunking_of_every_boundary():
    """Row c is the digest of exactly bytes [4096 c, 4096 (c + 1)): a payload built by concatenating
    known single-chunk messages reproduces their digests, and short last chunks hash only what is there."""
    for size in (1, 55, 56, 63, 64, 65, 4095, 4096, 4097, 8192, 8193):
        data = (np.arange(size, dtype=np.int64) * 7 + 3).astype(np.uint8)
        table = digest_table(data)
        assert table.shape == ((size + 4095) // 4096, 32)
        for c in range(table.shape[0]):
            piece = data[c * 4096:(c + 1) * 4096].tobytes()
            assert table[c].tobytes() == digest_table(piece)[0].tobytes()
    abc = digest_table(b"abc" + bytes(4093) + b"abc")
    assert abc[1].tobytes().hex() == KNOWN[b"abc"]
