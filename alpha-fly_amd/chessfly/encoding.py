"""Feature and policy-index constants the forward evaluator needs, and the from/to-square table of the
factorised policy head.

Only the numbers the network's input and output layers depend on live here; turning a python-chess board
into features (chessfly/encoding.py:25-52 in the reference) runs in the CPU search workers and is not part
of the evaluator.

Reference: chessfly/encoding.py:9-18 (sizes), :85-94 (move_squares).
"""

from __future__ import annotations

import numpy as np

# 12 piece planes (6 ours, 6 theirs) + en-passant plane = 13 x 64, then 4 castling rights, the halfmove clock
# and the repetition flag.  chessfly/encoding.py:9
N_BASE = 13 * 64 + 6
# + 64 squares we attack, 64 squares they attack, and "are we in check".  chessfly/encoding.py:10
N_FEATURES = N_BASE + 129
# from*64 + to (queen promotion implied) + 8 files x 3 directions x 3 underpromotion pieces.  chessfly/encoding.py:18
N_MOVES = 64 * 64 + 8 * 3 * 3


def move_squares() -> tuple[np.ndarray, np.ndarray]:
    """From- and to-square of every policy index, in the side-to-move frame (chessfly/encoding.py:85-94).

    Index i < 4096 is the pair (i // 64, i % 64).  Index 4096 + (file*3 + direction)*3 + piece is a pawn on
    the seventh rank (square 48 + file) underpromoting onto the eighth rank; direction 0/1/2 is a capture to
    the left / a straight push / a capture to the right, and the target file is clamped to the board.
    """
    idx = np.arange(N_MOVES, dtype=np.int64)
    frm = idx // 64
    to = idx % 64
    k = idx[4096:] - 4096
    file = k // 9
    direction = (k % 9) // 3
    frm[4096:] = 48 + file
    to[4096:] = 56 + np.clip(file + direction - 1, 0, 7)
    return frm, to
