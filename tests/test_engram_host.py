"""Host-side pieces of the Engram module, without a GPU: the token compression of smlm/engram.py:23-41
(NFKC-normalised lower-case text classes numbered in order of first appearance, byte pieces by their bytes,
vocabulary padding in classes of their own) on hand-made vocabularies, and the parameter names and initial state
a reference checkpoint expects (smlm/engram.py:76-117)."""
import torch

from smlm_hip.engram import EngramMemory, NgramHash, compress_vocab


def test_compression_merges_case_and_compatibility_forms():
    vocab = [b"Hello", b" the", b"hello", b"\xef\xbc\xa8ello", b"\xff", b" The", b"\xff", b"\xe2\x84\xa2"]
    ids, n = compress_vocab(vocab, 10)
    # "Hello" = "hello" = fullwidth-H "ello" (NFKC folds U+FF28 to H); " the" = " The"; the lone 0xff byte pieces
    # share their bytes; U+2122 (trade mark sign) becomes "tm" under NFKC and is new; ids 8, 9 are padding
    assert ids.tolist() == [0, 1, 0, 0, 2, 1, 2, 3, 4, 5]
    assert n == 6


def test_invalid_utf8_pieces_never_meet_text():
    # b"\xc3" alone is not UTF-8; its class must differ from any text class, including the text "\xc3" (U+00C3)
    ids, n = compress_vocab([b"\xc3", "Ã".encode(), b"\xc3"], 3)
    assert ids.tolist() == [0, 1, 0] and n == 2


def test_ngram_hash_buffers_and_pad_id():
    canon = torch.tensor([0, 1, 1, 2, 0])
    h = NgramHash(5, orders=(2, 3), heads=4, rows=97, seed=0, canon=canon)
    assert h.pad == 3 and h.history == 2 and h.n_lookups == 8
    assert h.mult.shape == (2, 4, 3) and bool((h.mult % 2 == 1).all()) and int(h.mult.max()) < 2 ** 31
    assert "mult" not in h.state_dict() and "canon" not in h.state_dict()
    assert torch.equal(NgramHash(5, (2, 3), 4, 97, seed=0, canon=canon).mult, h.mult)
    assert not torch.equal(NgramHash(5, (2, 3), 4, 97, seed=1, canon=canon).mult, h.mult)


def test_engram_state_dict_names_and_initial_state():
    m = EngramMemory(64, 16, 24, 53, conv_kernel=4, dilation=3)
    assert sorted(m.state_dict()) == sorted([
        "values.weight", "w_k.weight", "w_v.weight", "h_norm.weight", "k_norm.weight", "v_norm.weight",
        "conv.weight"])
    assert m.values.weight.shape == (16 * 53, 24) and m.past == 9
    assert not m.conv.weight.any()
    std = float(m.values.weight.std())
    assert abs(std - (16 * 24) ** -0.5) < 0.1 * (16 * 24) ** -0.5
