"""When to start the logits backward early (launch_early_backward).

A loss that knows d(loss)/d(logprobs) in closed form (the ClippedPG loss)
enqueues the logits backward for that gradient before autograd asks for it;
autograd's backward then compares the real upstream gradient with the one used
on the device and recomputes the whole gradient when they differ (a scaled
loss, a second consumer of the logprobs).  The guess costs nothing when it is
right and a wasted backward plus the redo when it is wrong, so the policy
follows the outcome of the last check:

``"adaptive"`` (the default) starts the backward early unless the last check
whose result has reached the host found a different gradient; after such a
miss the next ``retry_after`` opportunities run the plain backward instead (no
extra work), then speculation is tried again.  The check's flags are copied
to the host behind an event and read only once that copy has completed, so the
decision never waits for the GPU.  ``"always"`` speculates whenever the loss
allows it and ``"never"`` never does.  Results are bit-identical in all modes;
only the timing differs.  The policy is per process and shared by every call
site.
"""

from __future__ import annotations

from typing import Optional

import torch

from rl_amd import _C

MODES = ("adaptive", "always", "never")


class EarlyBackwardPolicy:
    def __init__(self, mode: str = "adaptive", retry_after: int = 16) -> None:
        self.configure(mode, retry_after)

    def configure(self, mode: str, retry_after: int = 16) -> None:
        if mode not in MODES:
            raise ValueError(f"early-backward mode must be one of {MODES}, got {mode!r}")
        if int(retry_after) < 0:
            raise ValueError(f"retry_after must be >= 0, got {retry_after}")
        self.mode = mode
        self.retry_after = int(retry_after)
        self.pending: Optional[list] = None  # start_fetch handle of the last check's flags
        self.skip = 0
        self.misses = 0  # checks that found a different gradient (read on the host)
        self.skipped = 0  # opportunities not taken after a miss

    def _drain(self) -> None:
        if self.pending is None:
            return
        flags = _C.poll_fetch(self.pending)
        if flags is None:
            return
        self.pending = None
        if any(flags):
            self.misses += 1
            self.skip = self.retry_after

    def should_launch(self) -> bool:
        """Whether an early backward should be started now (counts an opportunity)."""
        if self.mode == "never":
            return False
        if self.mode == "always":
            return True
        self._drain()
        if self.skip > 0:
            self.skip -= 1
            self.skipped += 1
            return False
        return True

    def checked(self, flags: torch.Tensor) -> None:
        """Record a device-side check (its flags tensor); read later without waiting."""
        if self.mode != "adaptive":
            return
        self._drain()
        # a newer check supersedes one whose copy has not completed yet
        self.pending = _C.start_fetch(flags)


POLICY = EarlyBackwardPolicy()


def set_early_backward(mode: str = "adaptive", retry_after: int = 16) -> None:
    """Choose when launch_early_backward starts the logits backward (see the module doc)."""
    POLICY.configure(mode, retry_after)


def early_backward_mode() -> str:
    return POLICY.mode
