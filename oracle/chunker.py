"""Oracle of the stream chunker that feeds the Token2Wav windows (``engine/token2wav_chunker.py:18-70``).

Codec tokens are buffered behind three silence tokens (4218); every time the buffer holds ``first_chunk`` (25 by default)
+ 3 tokens, those are a window and the buffer keeps all but the first ``first_chunk`` (later windows: 25); ``finish``
flushes the rest as the last window.  Pinned by the reference test's own restatement of the HF stream driver
(``tests/engine/test_token2wav_chunker.py:8-27``), which ``tests/test_oracle_chunker.py`` carries as a known-answer test.
"""

from __future__ import annotations

SILENCE_TOKEN = 4218
SILENCE_PREFIX = 3
PRE_LOOKAHEAD = 3
CHUNK = 25


def windows(tokens: list[int], step: int = 1, first_chunk: int = CHUNK) -> list[tuple[list[int], bool]]:
    """The windows a token-by-token (``step`` at a time) producer gets, then the final flush."""
    if not SILENCE_PREFIX < first_chunk <= CHUNK:
        raise ValueError("first_chunk out of range")
    buf = [SILENCE_TOKEN] * SILENCE_PREFIX
    emitted = 0
    out = []
    for i in range(0, len(tokens), step):
        for t in tokens[i:i + step]:
            buf.append(int(t))
            size = first_chunk if emitted == 0 else CHUNK
            if len(buf) >= size + PRE_LOOKAHEAD:
                out.append((buf[:size + PRE_LOOKAHEAD], False))
                emitted += 1
                buf = buf[size:]
    if buf:
        out.append((list(buf), True))
    return out
