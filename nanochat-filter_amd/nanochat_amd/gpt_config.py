"""Per-layer chunking of the look-back filters (reference
``nanochat/gpt_config.py:6-45``): ``ChunksAndHistory(p, q, k)``.

A look-back layer restarts its recurrence in chunks: the first chunk covers
the first ``p`` steps, every later chunk ``q`` steps, and each chunk is warmed
up over the ``k - 1`` steps before it.  ``p = UNBOUNDED_P`` is the full
recurrence (one chunk).  The rest of the reference's GPTConfig (attention
layout, LTV mode flags) is outside the filter path; the GPT harness has its
own config in ``gpt.py``.
"""

UNBOUNDED_P = 2_147_483_647


class ChunksAndHistory:
    def __init__(self, p: int, q: int, k: int):
        assert p >= 0, p
        assert q >= 1, q
        assert k >= 1, k
        self.p = p
        self.q = q
        self.k = k

    def deque_size(self) -> int:
        """States a KV cache keeps for chunk boundaries still ahead: the warm-ups
        that have started but not reached their chunk (``ceil((k - 1) / q)``)."""
        return 0 if self.is_unbounded() else (self.k - 1 + self.q - 1) // self.q

    def is_unbounded(self) -> bool:
        return self.p == UNBOUNDED_P

    def to_dict(self):
        return {"p": self.p, "q": self.q, "k": self.k}

    def to_comma_separated_str(self) -> str:
        return f"{self.p},{self.q},{self.k}"

    def __str__(self):
        return self.to_comma_separated_str()

    def __repr__(self):
        return f"ChunksAndHistory(p={self.p}, q={self.q}, k={self.k})"

    @classmethod
    def from_dict(cls, d):
        return cls(**d)


UNBOUNDED_LAYER_SPEC = ChunksAndHistory(p=UNBOUNDED_P, q=1, k=1)
