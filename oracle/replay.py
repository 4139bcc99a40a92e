"""Numpy restatement of the replay buffer's ring, n-step read and sampling.

Test infrastructure only: the product's replay never imports this.

ring            one array per leaf at (lane, column); column i holds the state
                its action was taken from; per-lane capacity ceil(capacity /
                n_envs) (ttrl/buffers/replay.py:62-129, :155-233)
sampleable      per lane start = pos if full else 0, count = (capacity if full
                else pos) - n_step, floored at 0 (ttrl/buffers/indexing.py:20-60)
n-step walk     g += disc * r; disc *= gamma in float64, stopping at the first
                `ends` (terminated or truncated) column; only `dones`
                (terminated) zeroes the bootstrap; steps = rewards summed
                (ttrl/buffers/indexing.py:94-131)
successor       the next column of the same lane, or the recorded final
                observation when the walk's last column ends its episode
                (ttrl/buffers/replaybatch.py:15-41)
batch           rewards = g as float32, dones = terminated, discounts =
                float32(gamma ** steps) (ttrl/buffers/replaybatch.py:44-76)
uniform draw    quota = rng.multinomial(batch, counts / total), then per lane
                rng.integers(0, count, size=k) (ttrl/buffers/samplers.py:86-109,
                ttrl/buffers/indexing.py:63-91)
priority draw   weights (p + eps) ** alpha in float64, fresh columns at the
                largest priority seen (initially 1); quota = rng.multinomial(
                batch, lane sums / total sum); per lane searchsorted(cumsum,
                rng.random(k) * cumsum[-1], 'right') capped at the run's end;
                IS weights (N P) ** -beta over the batch maximum, float32
                (ttrl/buffers/sampling.py:111-240)
"""

from __future__ import annotations

import numpy as np


class ReplayOracle:
    def __init__(self, obs_shape, obs_dtype, *, capacity: int, n_envs: int = 1, n_step: int = 1,
                 gamma: float = 0.99, seed=None, alpha: float | None = None, epsilon: float = 1e-6,
                 action_dim: int = 0):
        per_lane = -(-int(capacity) // int(n_envs))
        if per_lane <= n_step + 1:
            raise ValueError("ReplayOracle: a lane must hold more than n_step + 1 columns")
        self.n_envs, self.cols, self.n_step, self.gamma = int(n_envs), per_lane, int(n_step), float(gamma)
        L, C = self.n_envs, per_lane
        self.obs = np.zeros((L, C) + tuple(obs_shape), obs_dtype)
        # index actions, or float32 rows of action_dim for continuous actions
        self.actions = np.zeros((L, C, action_dim), np.float32) if action_dim else np.zeros((L, C), np.int64)
        self.rewards = np.zeros((L, C), np.float32)
        self.dones = np.zeros((L, C), bool)
        self.ends = np.zeros((L, C), bool)
        self.final = {}
        self.pos = np.zeros(L, np.int64)
        self.full = np.zeros(L, bool)
        self.rng = np.random.default_rng(seed)
        self.alpha, self.epsilon = alpha, float(epsilon)
        self.weight = np.zeros((L, C), np.float64) if alpha is not None else None
        self.max_priority = 1.0

    # -- writes --------------------------------------------------------------

    def add(self, lane, obs, action, reward, terminated, truncated=False, final_obs=None):
        col = int(self.pos[lane])
        self.final.pop((lane, col), None)
        self.obs[lane, col] = obs
        self.actions[lane, col] = action
        self.rewards[lane, col] = np.float32(reward)
        self.dones[lane, col] = bool(terminated)
        ended = bool(terminated) or bool(truncated)
        self.ends[lane, col] = ended
        if self.weight is not None:
            self.weight[lane, col] = (np.float64(self.max_priority) + self.epsilon) ** self.alpha
        if ended:
            self.final[(lane, col)] = np.array(final_obs, copy=True)
        nxt = (col + 1) % self.cols
        self.pos[lane] = nxt
        if nxt == 0:
            self.full[lane] = True

    def add_batch(self, obs, actions, rewards, terminated, truncated=None, final_obs=None):
        trunc = np.zeros(self.n_envs, bool) if truncated is None else np.asarray(truncated, bool)
        for lane in range(self.n_envs):
            ended = bool(terminated[lane]) or bool(trunc[lane])
            self.add(lane, obs[lane], actions[lane], rewards[lane], terminated[lane], trunc[lane],
                     final_obs[lane] if ended else None)

    # -- reads ---------------------------------------------------------------

    def sampleable(self):
        start = np.where(self.full, self.pos, 0)
        count = np.where(self.full, self.cols, self.pos) - self.n_step
        return start, np.maximum(count, 0)

    def walk(self, lanes, cols):
        g = np.zeros(len(cols), np.float64)
        disc = np.ones(len(cols), np.float64)
        end_cols = np.array(cols, np.int64)
        term = np.zeros(len(cols), bool)
        steps = np.zeros(len(cols), np.int64)
        for b, (lane, col) in enumerate(zip(lanes, cols)):
            for k in range(self.n_step):
                j = (col + k) % self.cols
                end_cols[b] = j
                g[b] += disc[b] * np.float64(self.rewards[lane, j])
                disc[b] *= self.gamma
                steps[b] += 1
                if self.ends[lane, j]:
                    term[b] = self.dones[lane, j]
                    break
        return g, end_cols, term, steps

    def successor(self, lane, end_col):
        if self.ends[lane, end_col]:
            return self.final[(lane, end_col)]
        return self.obs[lane, (end_col + 1) % self.cols]

    def assemble(self, lanes, cols, weights=None) -> dict:
        g, end_cols, term, steps = self.walk(lanes, cols)
        return dict(lanes=np.asarray(lanes, np.int64), cols=np.asarray(cols, np.int64),
                    obs=self.obs[lanes, cols], actions=self.actions[lanes, cols], rewards=g.astype(np.float32),
                    next_obs=np.stack([self.successor(l, e) for l, e in zip(lanes, end_cols)]),
                    dones=term.astype(np.float32), discounts=(self.gamma ** steps).astype(np.float32),
                    weights=weights)

    def sample(self, batch_size: int, beta: float | None = None) -> dict:
        start, count = self.sampleable()
        total = int(count.sum())
        if total <= 0:
            raise ValueError("ReplayOracle.sample: nothing sampleable")
        lanes_out, offs_out, probs = [], [], []
        if self.weight is None:
            quota = self.rng.multinomial(batch_size, count / total)
            for lane, k in enumerate(int(v) for v in quota):
                if k:
                    offs_out.append(self.rng.integers(0, int(count[lane]), size=k))
                    lanes_out.append(np.full(k, lane, np.int64))
            weights = None
        else:
            runs = [self.weight[l, (start[l] + np.arange(count[l])) % self.cols] for l in range(self.n_envs)]
            sums = np.array([w.sum() for w in runs], np.float64)
            quota = self.rng.multinomial(batch_size, sums / sums.sum())
            for lane, k in enumerate(int(v) for v in quota):
                if k:
                    cdf = np.cumsum(runs[lane])
                    picked = np.searchsorted(cdf, self.rng.random(k) * cdf[-1], side="right")
                    picked = np.minimum(picked, runs[lane].shape[0] - 1)
                    offs_out.append(picked)
                    lanes_out.append(np.full(k, lane, np.int64))
                    probs.append(runs[lane][picked] / sums.sum())
            w = (total * np.concatenate(probs)) ** (-float(beta))
            weights = (w / w.max()).astype(np.float32)
        lanes = np.concatenate(lanes_out)
        cols = (start[lanes] + np.concatenate(offs_out)) % self.cols
        return self.assemble(lanes, cols, weights)

    def update_priorities(self, lanes, cols, priorities):
        p = np.abs(np.asarray(priorities, np.float64).reshape(-1))
        self.weight[np.asarray(lanes), np.asarray(cols)] = (p + self.epsilon) ** self.alpha
        self.max_priority = max(self.max_priority, float(p.max()))
