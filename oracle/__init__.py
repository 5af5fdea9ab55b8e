"""CPU oracle for the logprob / ClippedPG / GRPO-advantage hot path.

TEST INFRASTRUCTURE ONLY.  This package restates the reference's algorithms
as plain PyTorch-on-CPU code, following the reference op sequence function by
function (each function cites the reference file:line it restates).  It is the
checker for the gfx950 kernels: only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and nothing in
``rl_amd`` does.

How each part is pinned (tests/test_oracle_*.py):
  * logprob.py   — closed forms: log_softmax + gather in float64, the
                   softmax-gradient identity sum_v grad = g * (1[t in range] - 1)
                   ... = 0, brute force on tiny vocabularies, chunk invariance.
  * loss.py      — the reference's 12 committed float64 golden cases
                   (tests/golden/clipped_pg_loss_goldens.json) at 1e-12, plus
                   the reference tests' hand-computed known answers.
  * advantage.py — known answers from the reference's unit tests
                   (baselines, stds, masked-reward advantages) and brute force.
  * sampling.py  — brute-force definitions on tiny vocabularies (every subset
                   checked against the top-k / nucleus definition) and the
                   reference's invariant checks.  The last-ulp rounding of CPU
                   torch softmax/cumsum at a top-p boundary is parity unpinned
                   (no frozen vectors exist in the reference for it); tie order
                   at the boundary follows a stable ascending sort.
"""
