"""Known-answer test of the stream chunker: the windows equal the HF stream driver as the reference's own test
restates it (``tests/engine/test_token2wav_chunker.py:8-27``), for the same token counts and producer step sizes."""

import pytest

from oracle import chunker


def hf_generator(tokens, chunk=25):
    i = 0
    while len(tokens) - i >= chunk:
        yield tokens[i:i + chunk], False
        i += chunk
    yield tokens[i:], True


def hf_driver(tokens, silence=True, pre_lookahead=3):
    buffer = [4218] * 3 if silence else []
    out = []
    for chunk, last in hf_generator(tokens):
        buffer += list(chunk)
        if len(buffer) >= 25 + pre_lookahead:
            out.append((buffer[: 25 + pre_lookahead], last))
            buffer = buffer[25:]
    if len(buffer) > 0:
        out.append((buffer, True))
    return out


@pytest.mark.parametrize("n", [0, 1, 24, 25, 26, 49, 50, 51, 137, 500])
@pytest.mark.parametrize("step", [1, 7, 25])
def test_windows_match_the_hf_driver(n, step):
    tokens = [(i * 37) % 4000 for i in range(n)]
    assert chunker.windows(tokens, step) == hf_driver(tokens)


@pytest.mark.parametrize("mutation", [{"silence": False}, {"pre_lookahead": 0}])
def test_mutations_are_detected(mutation):
    tokens = list(range(80))
    assert chunker.windows(tokens) != hf_driver(tokens, **mutation)


def test_first_chunk_ramp():
    toks = list(range(1, 81))
    ws = chunker.windows(toks, first_chunk=8)
    assert ws[0][0] == [4218] * 3 + toks[:8]
    assert all(len(w) == 28 for w, _ in ws[1:-1])
    decoded = [w[:-3] for w, _ in ws[:-1]] + [ws[-1][0]]
    assert [t for d in decoded for t in d] == [4218] * 3 + toks
