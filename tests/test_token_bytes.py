"""The token-bytes table of grammar-constrained sampling (Serve.swift:398-408:
each id decoded on its own, then UTF-8), for the byte-level tokenizer and for
an HF byte-level BPE tokenizer built in memory (no tokenizer file ships with
the reference)."""
import numpy as np
import pytest

from tinygpt_amd import grammar as G


def test_byte_level_table():
    # ByteTokenizer.decode (Tokenizer.swift:35-41) is UTF-8 decoding with
    # replacement: a lone byte >= 0x80 is an invalid sequence of its own
    t = G.token_bytes_table(300)
    assert len(t) == 300
    assert all(t[i] == bytes([i]) for i in range(128))
    assert all(t[i] == "�".encode() == b"\xef\xbf\xbd" for i in range(128, 256))
    assert all(t[i] == b"" for i in range(256, 300))
    # the table feeds the device row builder unchanged
    off, data = G.token_csr(t)
    assert off[-1] == 128 + 3 * 128 and data[off[200]:off[201]].tobytes() == b"\xef\xbf\xbd"


def test_byte_level_mask_rows_follow_the_table():
    # a grammar of ASCII letters: byte ids 128-255 decode to U+FFFD, whose
    # bytes are not letters, so no row allows them (as in the reference,
    # whose masker replays tokenBytes[id])
    d = G.compile_gbnf('root ::= [a-zA-Z]+')
    t = G.token_bytes_table(256)
    allowed = [i for i in range(256) if t[i] and d.walk(0, t[i]) >= 0]
    assert allowed == [i for i in range(256) if chr(i).isascii() and chr(i).isalpha()]


def _bpe():
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import decoders, models, pre_tokenizers

    # the GPT-2 byte-to-character map (printable bytes keep their character,
    # the others map to 256 + n in byte order)
    bs = list(range(0x21, 0x7F)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    cs, n = bs[:], 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    b2c = {b: chr(c) for b, c in zip(bs, cs)}
    vocab = {b2c[b]: b for b in range(256)}
    vocab[b2c[0xC3] + b2c[0xA9]] = 256  # "é" as one token
    tok = tokenizers.Tokenizer(models.BPE(vocab=vocab, merges=[(b2c[0xC3], b2c[0xA9])]))
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    tok.add_special_tokens(["<|eot|>"])
    return tok


def test_hf_bpe_table():
    tok = _bpe()
    V = tok.get_vocab_size()
    t = G.token_bytes_table(V, lambda ids: tok.decode(ids, skip_special_tokens=False))
    assert t[ord("a")] == b"a"
    assert t[256] == "é".encode() == b"\xc3\xa9"  # a whole character: its own bytes
    assert t[0xC3] == b"\xef\xbf\xbd"  # half of "é": U+FFFD, not 0xC3
    assert t[257] == b"<|eot|>"  # special tokens kept, as decode(tokens:) does
    assert tok.encode("aé").ids == [ord("a"), 256]
    # every entry is the id decoded alone, then UTF-8
    assert all(t[i] == tok.decode([i], skip_special_tokens=False).encode() for i in range(V))
