"""Learners on the MI355X path: DQN (double, n-step, prioritized weights)
and SAC (twin critics, learned temperature)."""
