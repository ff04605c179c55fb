"""CPU oracle for the MI355X learner hot path.

TEST INFRASTRUCTURE ONLY.  This package is a from-scratch CPU restatement (in
PyTorch, on the CPU) of the reference algorithm for one FlashSAC gradient
update and the PPO update.  It is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and never as the thing measured or shipped.  The product path
(``robolearn_amd``) never imports it and fails loudly when its HIP library is
missing.

Each function cites the reference file:line it follows.  Parity status of each
function (how it is pinned) is recorded in the module docstrings of
``oracle.flashsac``, ``oracle.ppo`` and ``oracle.optim``.
"""
