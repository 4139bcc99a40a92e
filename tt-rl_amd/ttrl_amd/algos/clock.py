"""The off-policy update clock: how many gradient steps the frames collected
so far are worth (ttrl/algos/clock.py:26-107).

Semantics kept from the reference, since they decide how much an agent
learns per frame: `train_freq` frames are worth one step, credit accrues
from the distance the frame number moved (so advancing twice to one frame
accrues once) and only past `warmup`, `skip` moves the frame without credit
(frames the buffer could not yet sample from owe nothing), `due`/`owed` only
read, `consume` keeps the remainder.

Held as an integer count of credited frames rather than a float sum of
fractions, so the owed count is exact however the frame increments divide
`train_freq`; the checkpoint form is the reference's {"frame", "credit"}
with credit in steps.
"""

from __future__ import annotations

__all__ = ["UpdateClock"]


class UpdateClock:
    def __init__(self, train_freq: int, warmup: int):
        if int(train_freq) < 1:
            raise ValueError(f"UpdateClock: train_freq must be >= 1, got {train_freq}")
        if int(warmup) < 0:
            raise ValueError(f"UpdateClock: warmup must be >= 0, got {warmup}")
        self.train_freq = int(train_freq)
        self.warmup = int(warmup)
        self._frame = 0
        self._credit_frames = 0  # credited frames not yet spent, train_freq per step

    def advance(self, frame: int) -> None:
        """Credit the frames between the last frame reached (or the warm-up
        end, whichever is later) and `frame`."""
        frame = int(frame)
        begin = max(self._frame, self.warmup)
        if frame > begin:
            self._credit_frames += frame - begin
        self._frame = max(self._frame, frame)

    def skip(self, frame: int) -> None:
        """Move to `frame` without credit."""
        self._frame = max(self._frame, int(frame))

    @property
    def due(self) -> bool:
        return self._credit_frames >= self.train_freq

    @property
    def owed(self) -> int:
        return self._credit_frames // self.train_freq

    def consume(self, steps: int) -> None:
        self._credit_frames -= int(steps) * self.train_freq

    def state_dict(self) -> dict:
        return {"frame": self._frame, "credit": self._credit_frames / self.train_freq}

    def load_state_dict(self, state: dict) -> None:
        self._frame = int(state["frame"])
        self._credit_frames = int(round(float(state["credit"]) * self.train_freq))
