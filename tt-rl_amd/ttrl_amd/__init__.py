"""ttrl_amd: tt-rl's learner-update path (engine, nets, DQN and SAC learners)
on AMD MI355X (gfx950) through hand-written HIP kernels in libttrl_hip.so."""

__version__ = "0.1.0"
