"""The tokenizer (host/Tokenizer.cpp through include/wsp_decoder.h), CPU only,
as Tests/Tokenizer/TokenizerTests.cpp checks the reference's: the reference's
own fixture vocabulary (Tests/Tokenizer/Fixtures/MiniTokenizer.json, kept as
tests/golden/mini_tokenizer.json) for merge order, repeated merges, byte round
trips, special tokens written in the text, and malformed documents; and the
byte layer, Unicode classes, UTF-8 edges and the pre-tokenizer split in a
sanitized native driver (tests/native/tokenizer_check.cpp)."""

import os
import subprocess

import pytest

from whispereacp_amd.tokenizer import Tokenizer, TokenizerError

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "mini_tokenizer.json")
E_ACUTE = "é"
NI_HAO = "你好世界"


@pytest.fixture(scope="module")
def tok():
    return Tokenizer.from_file(FIXTURE)


def test_fixture_loads(tok):
    assert tok.size() == 272
    assert tok.token_for_text("a") == ord("a")
    assert tok.token_for_text(b"\xc4\xa0the") == 261
    assert tok.token_for_text("nonesuch") == -1


def test_lower_rank_merges_win(tok):
    # "b c" is rank 0 and "a b" rank 1: "abc" is a + bc, never ab + c.
    assert tok.encode("abc") == [ord("a"), 256]
    assert tok.encode("ab") == [257]
    assert tok.encode("cab") == [ord("c"), 257]
    assert tok.encode("abcabc") == [ord("a"), 256, ord("a"), 256]


def test_merges_apply_repeatedly(tok):
    assert tok.encode("the") == [260]
    assert tok.encode(" the") == [261]
    # the vocabulary spells each byte's printable form with the byte's value as its id
    assert tok.encode("  the ") == [ord(" "), 261, ord(" ")]
    assert tok.encode("he") == [258]


def test_empty_input(tok):
    assert tok.encode("") == []
    assert tok.decode([]) == ""


def test_bytes_round_trip(tok):
    assert tok.encode(E_ACUTE) == [262]
    assert tok.encode("the" + E_ACUTE) == [260, 262]
    for text in ["the quick brown fox", "caf" + E_ACUTE + " " + NI_HAO, "\U0001F600 \U0001F44D"]:
        assert tok.decode(tok.encode(text)) == text
    assert tok.encode(b"\xff\xfe") == [0xFF, 0xFE]
    assert tok.encode(b"a\x80z") == [ord("a"), 0x80, ord("z")]
    assert tok.decode_bytes(tok.encode(b"\xff\xfe\x80\x01")) == b"\xff\xfe\x80\x01"
    every = bytes(range(1, 256))
    assert tok.decode_bytes(tok.encode(every)) == every


def test_special_tokens_in_text(tok):
    text = "<|startoftranscript|>abc<|endoftext|>"
    ids = tok.encode(text)
    assert ids == [264, ord("a"), 256, 263]
    assert tok.decode(ids) == "abc"
    assert tok.decode_keeping_special_tokens(ids) == text
    assert tok.is_special(263) and not tok.is_special(ord("a"))
    # an unknown <|...|> is ordinary text
    assert tok.decode(tok.encode("<|nope|>")) == "<|nope|>"
    # timestamps are added tokens too: decode skips them
    assert tok.decode([270, ord("a"), 271]) == "a"


def test_malformed_documents_are_refused():
    with pytest.raises(TokenizerError):
        Tokenizer.from_json_text("{ not json")
    with pytest.raises(TokenizerError, match="merges"):
        Tokenizer.from_json_text('{"model": {"vocab": {}}}')
    with pytest.raises(TokenizerError, match="no space"):
        Tokenizer.from_json_text('{"model": {"vocab": {"a": 0}, "merges": ["ab"]}}')
    with pytest.raises(TokenizerError):
        Tokenizer.from_file(os.path.join(HERE, "golden", "no_such_tokenizer.json"))


def test_merge_pairs_as_lists():
    tok = Tokenizer.from_json_text('{"model": {"vocab": {"a": 0, "b": 1, "ab": 2}, "merges": [["a", "b"]]}}')
    assert tok.encode("abab") == [2, 2]


def test_building_blocks_under_sanitizers():
    driver = os.path.join(HERE, "native", "_build", "tokenizer_check")
    if not os.path.exists(driver):
        subprocess.run(["make", "-s"], cwd=os.path.join(HERE, "native"), check=True)
    result = subprocess.run([driver, FIXTURE], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "failed: 0" in result.stdout and "read:" in result.stdout
