"""Fixtures and independent checks for the grammar-mask tests.

FAKE_VOCAB restates the reference's test vocabulary (GrammarTests.swift:7-27): the 256
single bytes, the multi-byte pieces listed there, and the end-of-turn id last (skipped by
the trie). DFAs are built by hand as [S][256] tables (-1 dead) with flags bit 0 accepting,
bit 1 consuming.
"""
from __future__ import annotations

import numpy as np

_PIECES = ["{\"", "\":", "\",", "\"}", "\": ", "\", \"", "true", "false", "null", "[\"", "\"]",
           "{}", "[]", "  ", "\n", "\n  ", "123", "12", "-1", "0.5", "e+", "name", "age",
           "Paris", "hello", " world", "<tool_call>", "</tool_call>", "<function=",
           "<parameter=", "</parameter>", "</function>", ">\n", "\n</parameter>\n", "é", "日本",
           "\\n", "\\\"", "the", " the", "city", "get_weather", "<think>", "</think>",
           "<|im_end|>"]
FAKE_VOCAB = [bytes([b]) for b in range(256)] + [s.encode("utf-8") for s in _PIECES]
FAKE_EOS = len(FAKE_VOCAB) - 1
FAKE_SKIP = np.zeros(len(FAKE_VOCAB), dtype=np.uint8)
FAKE_SKIP[FAKE_EOS] = 1

ACC, CON = 1, 2


def literal_dfa(text: bytes):
    """Accepts exactly `text`: state i has read text[:i]; the last state accepts only."""
    S = len(text) + 1
    nt = np.full((S, 256), -1, dtype=np.int32)
    for i, b in enumerate(text):
        nt[i, b] = i + 1
    fl = np.full(S, CON, dtype=np.uint8)
    fl[-1] = ACC
    return nt, fl


def digits_dfa():
    """One state: any run of ASCII digits, accepting."""
    nt = np.full((1, 256), -1, dtype=np.int32)
    nt[0, ord("0"):ord("9") + 1] = 0
    return nt, np.array([ACC | CON], dtype=np.uint8)


def object_int_dfa():
    """{"a": <integer>} with optional spaces after the colon (the ConstraintRowTests
    schema {"type":"object","properties":{"a":{"type":"integer"}},"required":["a"]},
    written as a DFA): 0 -{-> 1 -"-> 2 -a-> 3 -"-> 4 -:-> 5 (spaces), -?, digits, }."""
    nt = np.full((9, 256), -1, dtype=np.int32)
    for s, c, t in [(0, "{", 1), (1, "\"", 2), (2, "a", 3), (3, "\"", 4), (4, ":", 5),
                    (5, " ", 5), (5, "-", 6)]:
        nt[s, ord(c)] = t
    for d in range(ord("0"), ord("9") + 1):
        nt[5, d] = 7
        nt[6, d] = 7
        nt[7, d] = 7
    nt[7, ord("}")] = 8
    fl = np.full(9, CON, dtype=np.uint8)
    fl[8] = ACC
    return nt, fl


def random_vocab(rng, count: int, alphabet: int = 6, max_len: int = 40, p_empty=0.01,
                 p_dup=0.02):
    """Byte strings over a small alphabet (so that DFA transitions matter), with empty
    strings, duplicates and a length tail past 16 bytes."""
    toks = []
    for i in range(count):
        u = rng.random()
        if u < p_empty:
            toks.append(b"")
        elif u < p_empty + p_dup and toks:
            toks.append(toks[int(rng.integers(len(toks)))])
        else:
            n = int(min(max_len, 1 + rng.geometric(0.18)))
            toks.append(bytes((97 + rng.integers(alphabet, size=n)).astype(np.uint8).tolist()))
    return toks


def random_dfa(rng, S: int, alphabet: int = 6, p_dead: float = 0.15):
    """Transitions on the alphabet's bytes to random states or dead; other bytes dead."""
    nt = np.full((S, 256), -1, dtype=np.int32)
    sub = rng.integers(S, size=(S, alphabet)).astype(np.int32)
    sub[rng.random((S, alphabet)) < p_dead] = -1
    nt[:, 97:97 + alphabet] = sub
    fl = rng.integers(0, 4, size=S).astype(np.uint8)
    return nt, fl


class LazyTable:
    """The GrammarDFA interface (start, next, accepting, consuming; GrammarDFA.swift:13-58)
    over a full [S][256] table, as a host program that the device table interns from
    lazily; counts the transitions asked for."""

    def __init__(self, nt, fl, start=0):
        self.nt, self.fl, self.start = nt, fl, start
        self.calls = 0

    def next(self, s, b):
        self.calls += 1
        return int(self.nt[s, b])

    def accepting(self, s):
        return bool(self.fl[s] & ACC)

    def consuming(self, s):
        return bool(self.fl[s] & CON)


def brute_mask(tokens, width, eos, skip, nt, fl, key):
    """Per-token statement of the mask: token i (below width, non-empty, not skipped) is
    allowed iff its bytes never step to dead from a consuming state; end-of-turn ids join
    an accepting state; free and forced keys as DeviceMasks.all / only."""
    words = np.zeros((width + 31) // 32, dtype=np.uint32)

    def put(i):
        if 0 <= i < width:
            words[i >> 5] |= np.uint32(1 << (i & 31))

    if key == -1:
        for i in range(width):
            put(i)
        return words
    if key < -1:
        put(-2 - key)
        return words
    if key >= len(fl):
        return words
    if fl[key] & CON:
        for i, t in enumerate(tokens[:width]):
            if not t or (skip is not None and skip[i]):
                continue
            s = key
            for b in t:
                s = nt[s, b]
                if s < 0:
                    break
            if s >= 0:
                put(i)
    if fl[key] & ACC:
        for e in eos:
            put(e)
    return words


def bits(words, width):
    """Allowed ids of packed words."""
    w = np.asarray(words).view(np.uint32)
    return [i for i in range(width) if (int(w[i >> 5]) >> (i & 31)) & 1]
