"""Replay storage (ttrl/buffers): the GPU-resident replay buffer."""

from ttrl_amd.buffers.replay import DeviceBatch, PriorityConfig, ReplayBuffer, beta_at

__all__ = ["DeviceBatch", "PriorityConfig", "ReplayBuffer", "beta_at"]
