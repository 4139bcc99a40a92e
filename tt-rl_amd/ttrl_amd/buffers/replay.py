"""GPU-resident replay with n-step returns and prioritized sampling.

Same surface and semantics as ttrl/buffers/replay.py:58-282 with the
sampling of ttrl/buffers/samplers.py:86-125 and ttrl/buffers/sampling.py:
lanes are a real axis of the ring; column i of a lane holds the state its
action was taken from and the successor is the next column of the same lane,
or the episode-final observation of an ending column (the boundary table of
ttrl/buffers/boundaries.py); a transition is sampleable when its n-step window
and successor stay inside one lap (ttrl/buffers/indexing.py:20-60).

What moves to the device: the ring itself (one array per field, uint8 frames
stay uint8), the boundary observations (a pool of rows, allocated and
evicted on the host), the priority table and the running max priority, the
lane sums and the proportional pick of a prioritized draw, the
importance-sampling weights, the n-step walk, the batch assembly -- written
straight into a learner's bound input buffers when `out` names them -- and
the priority update from TD errors left on the device by the update.  What
stays on the host is everything that consumes the generator, in the
reference's order (the multinomial lane quota, then per lane the integer
offsets or the uniforms), so a seeded buffer draws the reference's
transitions; a prioritized draw reads its lane sums back for the quota.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.engine.tensor import DeviceArray, bound_block

__all__ = ["DeviceBatch", "PriorityConfig", "ReplayBuffer", "beta_at"]

PICK_CHUNK = 1024  # run positions per chunk sum of a prioritized draw


@dataclass(frozen=True)
class PriorityConfig:
    """Prioritized replay's settings (ttrl/buffers/sampling.py:58-100)."""

    alpha: float = 0.6
    beta_start: float = 0.4
    beta_end: float = 1.0
    beta_anneal_updates: int = 1_000_000
    epsilon: float = 1e-6

    def __post_init__(self):
        if not 0.0 <= self.alpha <= 1.0:
            raise ValueError(f"PriorityConfig: alpha must be in [0, 1], got {self.alpha}")
        for name in ("beta_start", "beta_end"):
            value = getattr(self, name)
            if not 0.0 <= value <= 1.0:
                raise ValueError(f"PriorityConfig: {name} must be in [0, 1], got {value}")
        if self.beta_anneal_updates < 1:
            raise ValueError(f"PriorityConfig: beta_anneal_updates must be >= 1, got {self.beta_anneal_updates}")
        if self.epsilon <= 0.0:
            raise ValueError(f"PriorityConfig: epsilon must be > 0, got {self.epsilon}")


def beta_at(cfg: PriorityConfig, update: int) -> float:
    """The annealed beta at a gradient-step count, linear then held
    (ttrl/buffers/sampling.py:103-106)."""
    frac = min(1.0, max(0, int(update)) / cfg.beta_anneal_updates)
    return cfg.beta_start + frac * (cfg.beta_end - cfg.beta_start)


@dataclass
class DeviceBatch:
    """One sampled batch, on the device (ttrl/buffers/types.py:50-76).
    `lanes` and `cols` are device int32 arrays; `host()` reads everything."""

    obs: DeviceArray
    next_obs: DeviceArray
    actions: DeviceArray
    rewards: DeviceArray
    dones: DeviceArray
    discounts: DeviceArray
    weights: DeviceArray | None
    lanes: DeviceArray
    cols: DeviceArray
    actions_onehot: DeviceArray | None = None

    def host(self) -> dict:
        out = {k: getattr(self, k).numpy() for k in ("obs", "next_obs", "actions", "rewards", "dones", "discounts",
                                                      "lanes", "cols")}
        out["weights"] = None if self.weights is None else self.weights.numpy()
        return out


class _PriorityWords:
    """One mapped host block of a prioritized draw: run starts and counts
    (int32 per lane), lane sums (float64 per lane), the batch's lanes (int32)
    and uniforms (float64), as numpy views and device addresses."""

    def __init__(self, dev, lanes: int, max_batch: int):
        layout, off = {}, 0
        for name, n, dt in (("start", lanes, np.int32), ("count", lanes, np.int32), ("sums", lanes, np.float64),
                            ("lanes", max_batch, np.int32), ("u", max_batch, np.float64)):
            off = -(-off // 64) * 64
            layout[name] = (off, n, dt)
            off += n * np.dtype(dt).itemsize
        self.block = dev.mapped_block(off)
        for name, (o, n, dt) in layout.items():
            setattr(self, name, self.block.view(o, (n,), dt))
            setattr(self, "d_" + name, self.block.dptr + o)


class ReplayBuffer:
    """Uniform or prioritized off-policy replay with n-step returns over
    `n_envs` lanes, resident in device memory."""

    def __init__(self, obs_spec, action_spec, device, *, capacity: int, n_envs: int = 1, n_step: int = 1,
                 gamma: float = 0.99, seed: int | None = None, priority: PriorityConfig | None = None,
                 boundary_rows: int | None = None, max_batch: int = 1024):
        if n_envs < 1:
            raise ValueError(f"ReplayBuffer: n_envs must be >= 1, got {n_envs}")
        if n_step < 1:
            raise ValueError(f"ReplayBuffer: n_step must be >= 1, got {n_step}")
        if not 0.0 < gamma <= 1.0:
            raise ValueError(f"ReplayBuffer: gamma must be in (0, 1], got {gamma}")
        per_lane = -(-int(capacity) // int(n_envs))
        if per_lane <= n_step + 1:
            raise ValueError(
                f"ReplayBuffer: capacity {capacity} split across {n_envs} lanes gives {per_lane} columns per "
                f"lane, but one transition reads n_step + 1 = {n_step + 1} columns of its own lane, so a lane "
                f"that short has no sampleable transition. Raise capacity or lower n_envs.")
        if action_spec.kind not in ("discrete", "continuous"):
            raise ValueError(f"ReplayBuffer: unsupported action kind {action_spec.kind!r}")
        # discrete actions are stored as indices, continuous ones as float32 rows
        self.action_dim = int(action_spec.dim) if action_spec.kind == "continuous" else 0
        self.obs_spec, self.action_spec, self.device = obs_spec, action_spec, device
        self.n_envs, self.per_lane_capacity = int(n_envs), per_lane
        self.capacity = per_lane * self.n_envs
        self.n_step, self.gamma = int(n_step), float(gamma)
        self.priority = priority
        if obs_spec.kind == "image":
            self.obs_shape, self.obs_dtype = tuple(obs_spec.shape), np.dtype(np.uint8)
        else:
            self.obs_shape, self.obs_dtype = (int(obs_spec.size),), np.dtype(np.float32)
        self.obs_bytes = int(np.prod(self.obs_shape)) * self.obs_dtype.itemsize
        L, Cc, dev = self.n_envs, per_lane, device
        cells = L * Cc
        self._obs = DeviceArray(dev, (cells * self.obs_bytes,), np.uint8)
        self._actions = DeviceArray(dev, (cells,), np.int32)
        self._action_vec = DeviceArray(dev, (cells * self.action_dim,), np.float32) if self.action_dim else None
        self._rewards = DeviceArray(dev, (cells,), np.float32)
        self._flags = DeviceArray(dev, (2 * cells,), np.uint8)  # dones | ends
        self._final_slot = DeviceArray(dev, (cells,), np.int32)
        self._final_slot.fill(-1)
        rows = int(boundary_rows) if boundary_rows is not None else max(64, cells // 16)
        self._final_rows = rows
        self._final_obs = DeviceArray(dev, (max(rows, 1) * self.obs_bytes,), np.uint8)
        self._free_rows = list(range(rows - 1, -1, -1))
        self._row_of: dict[tuple[int, int], int] = {}
        self._weight = self._max_priority = None
        if priority is not None:
            self._weight = DeviceArray(dev, (cells,), np.float64)
            self._weight.upload(np.zeros(cells))
            self._max_priority = DeviceArray(dev, (1,), np.float64)
            self._max_priority.upload(np.ones(1))
        self._ring = _lib.ReplayRing(
            L, Cc, self.obs_bytes, self._obs.ptr, self._actions.ptr, self._rewards.ptr, self._flags.ptr,
            self._flags.ptr + cells, self._final_slot.ptr, self._final_obs.ptr, rows,
            None if self._weight is None else self._weight.ptr,
            None if self._max_priority is None else self._max_priority.ptr,
            0.0 if priority is None else float(priority.alpha), 1e-6 if priority is None else float(priority.epsilon),
            None if self._action_vec is None else self._action_vec.ptr, self.action_dim)
        self._pos = np.zeros(L, np.int64)
        self._full = np.zeros(L, bool)
        self._rng = np.random.default_rng(seed)
        # Staging of one vector-env step's writes, and of one draw.
        self._stage_in, self._stage = bound_block(dev, self._stage_specs(L, True))
        self._stage_host = np.zeros(self._stage.nbytes, np.uint8)
        self.max_batch = int(max_batch)
        self._max_chunks = -(-Cc // PICK_CHUNK)
        self._draw_in, self._draw = bound_block(dev, [
            ("lanes", np.zeros(self.max_batch, np.int32)), ("cols", np.zeros(self.max_batch, np.int32)),
            ("u", np.zeros(self.max_batch, np.float64)), ("start", np.zeros(L, np.int32)),
            ("count", np.zeros(L, np.int32))])
        self._draw_host = np.zeros(self._draw.nbytes, np.uint8)
        if priority is not None:
            self._csum = DeviceArray(dev, (L * self._max_chunks,), np.float64)
            self._picked = DeviceArray(dev, (self.max_batch,), np.float64)
            # The words a prioritized draw exchanges between host and kernels
            # (run extents, lane sums, the generator's lanes and uniforms), in
            # two mapped host blocks used in turn: the kernels read and write
            # them in place, and a draw never rewrites the block the previous
            # draw's kernels may still read (each draw waits for its lane sums,
            # which follow the previous draw's kernels on the stream).
            self._pm = [_PriorityWords(dev, L, self.max_batch) for _ in range(2)]
            self._pm_next = 0
            self._lane_ids = np.arange(L, dtype=np.int32)
            self._draw_cache: dict = {}
        self._last = None  # (n, device lanes, device cols) of the last draw

    # -- size ----------------------------------------------------------------

    @property
    def size(self) -> int:
        return int(np.where(self._full, self.per_lane_capacity, self._pos).sum())

    def _sampleable(self):
        start = np.where(self._full, self._pos, 0)
        count = np.where(self._full, self.per_lane_capacity, self._pos) - self.n_step
        return start, np.maximum(count, 0)

    @property
    def num_sampleable(self) -> int:
        return int(self._sampleable()[1].sum())

    @property
    def num_boundaries(self) -> int:
        return len(self._row_of)

    @property
    def prioritized(self) -> bool:
        return self.priority is not None

    # -- writing -------------------------------------------------------------

    def _obs_rows(self, obs, n: int, what: str) -> np.ndarray:
        arr = np.asarray(obs)
        if arr.dtype != self.obs_dtype:
            raise ValueError(f"ReplayBuffer.{what}: observations are {self.obs_dtype}, got {arr.dtype}")
        if arr.shape != (n,) + self.obs_shape:
            raise ValueError(f"ReplayBuffer.{what}: expected observations of shape {(n,) + self.obs_shape}, "
                             f"got {arr.shape}")
        return arr

    def _write(self, lanes, obs, actions, rewards, term, ended, final_obs) -> None:
        """Entries in write order: lanes[e] may repeat (successive steps of a
        lane), each taking that lane's next column."""
        lanes = np.asarray(lanes, np.int64)
        n = len(lanes)
        cols = np.empty(n, np.int64)
        pos = self._pos.copy()
        full = self._full.copy()
        for e, lane in enumerate(lanes):
            cols[e] = pos[lane]
            nxt = (int(pos[lane]) + 1) % self.per_lane_capacity
            pos[lane] = nxt
            full[lane] |= nxt == 0
        frow = np.full(n, -1, np.int32)
        ended = np.asarray(ended, bool)
        if self._row_of or ended.any():
            for e in range(n):
                key = (int(lanes[e]), int(cols[e]))
                old = self._row_of.pop(key, None)  # evict the overwritten lap's boundary first
                if old is not None:
                    self._free_rows.append(old)
                if ended[e]:
                    if not self._free_rows:
                        raise RuntimeError(
                            f"ReplayBuffer: the boundary pool holds {self._final_rows} episode-final observations "
                            f"and all are live; build the buffer with a larger boundary_rows")
                    row = self._free_rows.pop()
                    self._row_of[key] = row
                    frow[e] = row
        with_final = final_obs is not None and ended.any()
        if n <= self.n_envs:
            stage, block, host = self._stage_in, self._stage, self._stage_host
        else:
            stage, block = self._staging(n, with_final)
            host = np.zeros(block.nbytes, np.uint8)
        host[:] = 0
        if self.action_dim:
            acts = np.asarray(actions, np.float32).reshape(n, self.action_dim)
        else:
            acts = np.asarray(actions).reshape(-1)
            if acts.dtype.kind == "f" and np.any(acts != np.floor(acts)):
                raise ValueError("ReplayBuffer: a discrete action must be a whole number")
            acts = acts.astype(np.int32)
        fields = [("lane", lanes.astype(np.int32)), ("col", cols.astype(np.int32)),
                  ("action", acts), ("reward", np.asarray(rewards, np.float32)),
                  ("term", np.asarray(term, np.uint8)), ("end", ended.astype(np.uint8)), ("frow", frow),
                  ("obs", obs)]
        if with_final:
            fields.append(("final", final_obs))
        for name, arr in fields:
            view = stage[name]
            a = np.ascontiguousarray(arr).reshape(-1).view(np.uint8)
            off = view.offset - block.offset
            host[off:off + a.nbytes] = a
        block.upload(host)
        final = stage["final"] if "final" in stage else stage["obs"]  # read only for rows with a boundary
        vec = bool(self.action_dim)
        self.device.call("ttrl_replay_write", C.byref(self._ring), n, stage["lane"].vp, stage["col"].vp,
                         None if vec else stage["action"].vp, stage["action"].vp if vec else None,
                         stage["reward"].vp, stage["term"].vp, stage["end"].vp, stage["frow"].vp, stage["obs"].vp,
                         final.vp)
        self._pos, self._full = pos, full

    def _stage_specs(self, n: int, with_final: bool):
        action = np.zeros((n, self.action_dim), np.float32) if self.action_dim else np.zeros(n, np.int32)
        specs = [("lane", np.zeros(n, np.int32)), ("col", np.zeros(n, np.int32)), ("action", action),
                 ("reward", np.zeros(n, np.float32)), ("term", np.zeros(n, np.uint8)), ("end", np.zeros(n, np.uint8)),
                 ("frow", np.zeros(n, np.int32)), ("obs", np.zeros(n * self.obs_bytes, np.uint8))]
        if with_final:
            specs.append(("final", np.zeros(n * self.obs_bytes, np.uint8)))
        return specs

    def _staging(self, n: int, with_final: bool):
        return bound_block(self.device, self._stage_specs(n, with_final))

    def add_steps(self, obs, actions, rewards, terminated, truncated=None, final_obs=None) -> None:
        """T vector-env steps at once, every argument [T, n_envs, ...]: the
        same as T successive add_batch calls, in one upload and one launch.
        final_obs, when given, is [T, n_envs, ...] with the ending entries'
        final observations (other rows are ignored)."""
        obs = np.asarray(obs)
        T, L = obs.shape[0], self.n_envs
        rows = self._obs_rows(obs.reshape((T * L,) + obs.shape[2:]), T * L, "add_steps")
        term = np.asarray(terminated, bool).reshape(T * L)
        trunc = np.zeros(T * L, bool) if truncated is None else np.asarray(truncated, bool).reshape(T * L)
        ended = term | trunc
        fin = None
        if ended.any():
            if final_obs is None:
                raise ValueError("ReplayBuffer.add_steps: some lanes ended but final_obs is None")
            fin = np.asarray(final_obs, self.obs_dtype).reshape((T * L,) + self.obs_shape)
        self._write(np.tile(np.arange(L), T), rows, np.asarray(actions).reshape(-1),
                    np.asarray(rewards).reshape(-1), term, ended, fin)

    def add(self, obs, action, reward, terminated: bool, truncated: bool = False, *, final_obs=None,
            lane: int = 0) -> None:
        """One transition into one lane (ttrl/buffers/replay.py:155-168)."""
        if not 0 <= lane < self.n_envs:
            raise ValueError(f"ReplayBuffer.add: lane must be in [0, {self.n_envs}), got {lane}")
        ended = bool(terminated) or bool(truncated)
        if ended and final_obs is None:
            raise ValueError(f"ReplayBuffer.add: lane {lane} ended but final_obs is None")
        if not ended and final_obs is not None:
            raise ValueError(f"ReplayBuffer.add: lane {lane} did not end but final_obs was given")
        rows = self._obs_rows(np.asarray(obs)[None], 1, "add")
        fin = None if final_obs is None else self._obs_rows(np.asarray(final_obs)[None], 1, "add")
        self._write(np.array([lane]), rows, [action], [reward], [bool(terminated)], [ended], fin)

    def add_lanes(self, lanes, obs, actions, rewards, terminated, truncated=None, final_obs=None) -> None:
        """One transition into each of `lanes` (distinct), in one upload and
        one launch: the lanes of a vector-env step that are real transitions
        (ttrl/algos/offpolicy.py:37-58 writes them one `add` at a time).
        Arguments are lane-major over `lanes`; final_obs rows are read for
        the entries that ended."""
        lanes = np.asarray(lanes, np.int64).reshape(-1)
        n = lanes.size
        if n == 0:
            return
        if np.unique(lanes).size != n or lanes.min() < 0 or lanes.max() >= self.n_envs:
            raise ValueError(f"ReplayBuffer.add_lanes: lanes must be distinct and in [0, {self.n_envs}), "
                             f"got {lanes.tolist()}")
        rows = self._obs_rows(np.asarray(obs).reshape((n,) + self.obs_shape), n, "add_lanes")
        term = np.asarray(terminated, bool).reshape(n)
        trunc = np.zeros(n, bool) if truncated is None else np.asarray(truncated, bool).reshape(n)
        ended = term | trunc
        fin = None
        if ended.any():
            if final_obs is None:
                raise ValueError("ReplayBuffer.add_lanes: some lanes ended but final_obs is None")
            fin = np.asarray(final_obs, self.obs_dtype).reshape((n,) + self.obs_shape)
        self._write(lanes, rows, actions, np.asarray(rewards).reshape(-1), term, ended, fin)

    def add_batch(self, obs, actions, rewards, terminated, truncated=None, final_obs=None) -> None:
        """One vector-env step, the leading axis of every argument the lane
        (ttrl/buffers/replay.py:170-187, ttrl/buffers/writes.py:38-70)."""
        L = self.n_envs
        rows = self._obs_rows(obs, L, "add_batch")
        term = np.asarray(terminated, bool).reshape(-1)
        trunc = np.zeros(L, bool) if truncated is None else np.asarray(truncated, bool).reshape(-1)
        ended = term | trunc
        if ended.any() and final_obs is None:
            raise ValueError(f"ReplayBuffer.add_batch: lanes {np.flatnonzero(ended).tolist()} ended but "
                             f"final_obs is None")
        fin = np.zeros((L,) + self.obs_shape, self.obs_dtype)
        for lane in np.flatnonzero(ended):
            f = final_obs[lane]
            if f is None:
                raise ValueError(f"ReplayBuffer.add_batch: lane {lane} ended but its final_obs is None")
            fin[lane] = np.asarray(f, self.obs_dtype).reshape(self.obs_shape)
        self._write(np.arange(L), rows, np.asarray(actions).reshape(-1), np.asarray(rewards).reshape(-1), term,
                    ended, fin)

    # -- sampling ------------------------------------------------------------

    def _draw_put(self, name: str, array) -> None:
        view = self._draw_in[name]
        arr = np.ascontiguousarray(array, dtype=view.dtype).reshape(-1).view(np.uint8)
        off = view.offset - self._draw.offset
        self._draw_host[off:off + arr.nbytes] = arr

    def sample(self, batch_size: int, *, beta: float | None = None, out: dict | None = None) -> DeviceBatch:
        """One batch (ttrl/buffers/replay.py:254-282).  `out` may name
        destination device arrays (obs, next_obs, actions_onehot, rewards,
        dones, discounts, weights), e.g. a learner's bound inputs."""
        if batch_size < 1:
            raise ValueError(f"ReplayBuffer.sample: batch_size must be >= 1, got {batch_size}")
        if batch_size > self.max_batch:
            raise ValueError(f"ReplayBuffer.sample: batch_size {batch_size} exceeds max_batch {self.max_batch}")
        start, count = self._sampleable()
        total = int(count.sum())
        if total <= 0:
            raise ValueError(f"ReplayBuffer.sample: no lane holds a complete {self.n_step}-step window and its "
                             f"successor observation yet (size={self.size}); gate on num_sampleable")
        weights = None
        if self.priority is None:
            if beta is not None:
                raise ValueError("ReplayBuffer.sample: beta was given but this buffer samples uniformly, so there "
                                 "is no sampling bias for an importance-sampling weight to correct.")
            quota = self._rng.multinomial(batch_size, count / total)
            lanes, offs = [], []
            for lane, k in enumerate(int(v) for v in quota):
                if k:
                    offs.append(self._rng.integers(0, int(count[lane]), size=k))
                    lanes.append(np.full(k, lane, np.int64))
            lanes = np.concatenate(lanes)
            cols = (start[lanes] + np.concatenate(offs)) % self.per_lane_capacity
            self._draw_put("lanes", lanes)
            self._draw_put("cols", cols)
            self._draw.upload(self._draw_host)
        else:
            if beta is None:
                raise ValueError("ReplayBuffer.sample: this buffer samples by priority, so the batch's "
                                 "importance-sampling weights need a beta (beta_at(cfg, update_count)).")
            return self._sample_prioritized(batch_size, start, count, total, beta, out)
        return self._assemble(batch_size, out, weights)

    def _sample_prioritized(self, n: int, start, count, total: int, beta: float, out) -> DeviceBatch:
        """The lane sums computed into a mapped block and waited for, the
        generator's draws in the reference's order (the multinomial lane
        quota, then each lane's uniforms), then the pick, the IS weights and
        the assembly enqueued by one call that reads the draws in place
        (ttrl/buffers/sampling.py:195-240)."""
        dev = self.device
        w = self._pm[self._pm_next]
        self._pm_next ^= 1
        w.start[:] = start
        w.count[:] = count
        dev.call("ttrl_replay_lane_sums", C.byref(self._ring), C.c_void_p(w.d_start), C.c_void_p(w.d_count),
                 PICK_CHUNK, self._max_chunks, self._csum.vp, C.c_void_p(w.d_sums))
        dev.synchronize()
        sums = w.sums.copy()
        if not np.all(np.isfinite(sums)):
            # A non-finite TD error written by update_priorities_device
            # (the host path refuses it on entry) poisons its lane's sum.
            raise ValueError("ReplayBuffer.sample: a priority is NaN or infinite (written by a device "
                             "priority update since the last sample)")
        if sums.sum() <= 0.0:
            raise RuntimeError(f"replay: {total} transitions are sampleable but every priority in the "
                               f"sampleable runs is zero")
        quota = self._rng.multinomial(n, sums / sums.sum())
        # each lane's uniforms in lane order: one call draws the same
        # sequence as one call per lane
        w.lanes[:n] = np.repeat(self._lane_ids, quota)
        w.u[:n] = self._rng.random(n)
        desc, batch = self._draw_desc(w, n, out)
        desc.total_count = total
        desc.beta = float(beta)
        dev.call("ttrl_replay_draw_batch", C.byref(self._ring), C.byref(desc))
        self._last = n
        return batch

    def _draw_desc(self, w, n: int, out):
        """The draw call's arguments and the batch it returns, for mapped
        block w, batch size n and the destinations `out` names, kept for the
        next draw of the same shape into the same arrays."""
        key = (id(w), n, None if not out else tuple((k, v.ptr) for k, v in out.items()))
        hit = self._draw_cache.get(key)
        if hit is not None:
            return hit
        dev = self.device
        dst = self._outputs(n, out)
        weights = (out or {}).get("weights") or DeviceArray(dev, (n, 1))
        d = self._draw_in
        desc = _lib.ReplayDraw(
            n=n, lane=w.d_lanes, lanes_out=d["lanes"].ptr, u=w.d_u, start=w.d_start, count=w.d_count,
            chunk=PICK_CHUNK, max_chunks=self._max_chunks, chunk_sums=self._csum.ptr, sums=w.d_sums,
            total_count=0, beta=0.0, cols_out=d["cols"].ptr, picked_weight=self._picked.ptr,
            weights_out=weights.ptr, n_step=self.n_step, gamma=self.gamma, obs_out=dst["obs"].ptr,
            next_obs_out=dst["next_obs"].ptr, actions_onehot=None if dst["onehot"] is None else dst["onehot"].ptr,
            num_actions=dst["A"], actions_out=None if self.action_dim else dst["actions"].ptr,
            action_vec_out=dst["actions"].ptr if self.action_dim else None, rewards_out=dst["rewards"].ptr,
            dones_out=dst["dones"].ptr, discounts_out=dst["discounts"].ptr)
        batch = DeviceBatch(dst["obs"], dst["next_obs"], dst["actions"], dst["rewards"], dst["dones"],
                            dst["discounts"], weights, d["lanes"].view(0, (n,)), d["cols"].view(0, (n,)),
                            dst["onehot"])
        if len(self._draw_cache) >= 16:
            self._draw_cache.clear()
        self._draw_cache[key] = (desc, batch)
        return desc, batch

    def _outputs(self, n: int, out: dict | None) -> dict:
        """The batch's destination arrays: out's where given, else new."""
        dev, out = self.device, dict(out or {})
        A = int(self.action_spec.n) if not self.action_dim else 0

        def dst(name, shape, dtype=np.float32):
            a = out.get(name)
            if a is None:
                return DeviceArray(dev, shape, dtype)
            if a.nbytes != int(np.prod(shape)) * np.dtype(dtype).itemsize:
                raise ValueError(f"ReplayBuffer.sample: out[{name!r}] holds {a.nbytes} bytes, the batch needs "
                                 f"{int(np.prod(shape)) * np.dtype(dtype).itemsize}")
            return a

        obs = dst("obs", (n,) + self.obs_shape, self.obs_dtype)
        nxt = dst("next_obs", (n,) + self.obs_shape, self.obs_dtype)
        onehot = out.get("actions_onehot")
        if self.action_dim:
            onehot = None
            actions = dst("actions", (n, self.action_dim))
        else:
            if onehot is not None:
                onehot = dst("actions_onehot", (n, A))
            actions = DeviceArray(dev, (n,), np.int32)
        rewards, dones, discounts = (dst(k, (n, 1)) for k in ("rewards", "dones", "discounts"))
        return {"obs": obs, "next_obs": nxt, "onehot": onehot, "A": A, "actions": actions, "rewards": rewards,
                "dones": dones, "discounts": discounts}

    def _assemble(self, n: int, out: dict | None, weights) -> DeviceBatch:
        o = self._outputs(n, out)
        d = self._draw_in
        onehot, actions = o["onehot"], o["actions"]
        self.device.call("ttrl_replay_assemble", C.byref(self._ring), n, d["lanes"].vp, d["cols"].vp, self.n_step,
                         C.c_double(self.gamma), o["obs"].vp, o["next_obs"].vp,
                         None if onehot is None else onehot.vp, o["A"], None if self.action_dim else actions.vp,
                         actions.vp if self.action_dim else None, o["rewards"].vp, o["dones"].vp,
                         o["discounts"].vp)
        self._last = n
        return DeviceBatch(o["obs"], o["next_obs"], actions, o["rewards"], o["dones"], o["discounts"], weights,
                           d["lanes"].view(0, (n,)), d["cols"].view(0, (n,)), onehot)

    # -- priorities ----------------------------------------------------------

    def update_priorities(self, lanes, cols, priorities) -> None:
        """Record TD errors by (lane, column) (ttrl/buffers/replay.py:233-252,
        ttrl/buffers/sampling.py:168-193).  Host arrays."""
        if not self.prioritized:
            raise ValueError("ReplayBuffer.update_priorities: this buffer samples uniformly, so a priority would "
                             "be stored and never read. Build it with priority=PriorityConfig(...).")
        lanes = np.asarray(lanes).reshape(-1)
        cols = np.asarray(cols).reshape(-1)
        p = np.asarray(priorities, np.float64).reshape(-1)
        if p.shape != lanes.shape or cols.shape != lanes.shape:
            raise ValueError(f"ReplayBuffer.update_priorities: {p.shape[0]} priorities for {lanes.shape[0]} "
                             f"sampled transitions; one per sampled transition")
        if not np.all(np.isfinite(p)):
            raise ValueError("ReplayBuffer.update_priorities: a priority is NaN or infinite")
        n = lanes.shape[0]
        if n > self.max_batch:
            raise ValueError(f"ReplayBuffer.update_priorities: {n} entries exceed max_batch {self.max_batch}")
        if np.any((lanes < 0) | (lanes >= self.n_envs) | (cols < 0) | (cols >= self.per_lane_capacity)):
            raise ValueError("ReplayBuffer.update_priorities: a (lane, column) lies outside the ring")
        self._draw_put("lanes", lanes)
        self._draw_put("cols", cols)
        self._draw.upload(self._draw_host)
        prio = DeviceArray(self.device, (n,), np.float64)  # float64 end to end, as the reference
        prio.upload(p)
        d = self._draw_in
        self.device.call("ttrl_replay_update_priorities_f64", C.byref(self._ring), n, d["lanes"].vp, d["cols"].vp,
                         prio.vp)

    def update_priorities_device(self, batch: DeviceBatch, priorities: DeviceArray) -> None:
        """The priority update of the last sampled batch from TD errors that
        are already on the device (no host transfer).  Call it before the
        next `add`, as the reference's update_priorities."""
        if not self.prioritized:
            raise ValueError("ReplayBuffer.update_priorities_device: this buffer samples uniformly")
        n = batch.lanes.numel
        if priorities.numel != n:
            raise ValueError(f"ReplayBuffer.update_priorities_device: {priorities.numel} priorities for {n} rows")
        self.device.call("ttrl_replay_update_priorities", C.byref(self._ring), n, batch.lanes.vp, batch.cols.vp,
                         priorities.vp)

    # -- inspection (tests) ----------------------------------------------------

    def priorities_numpy(self) -> np.ndarray:
        """The (lanes, cols) weight table, float64 (a host read)."""
        return self._weight.numpy().reshape(self.n_envs, self.per_lane_capacity)
