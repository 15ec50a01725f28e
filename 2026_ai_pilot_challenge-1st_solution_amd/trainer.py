"""PPOGPUTrainer's collection and update entry points (research/competition_36500/runtime/
cuda_fdm/ppo_gpu.py:1098-1183, 1856-2145) over this package's collector and updater, so that the
reference's training loop can call ``collect_rollout(opp_kind="pool", frozen_opp=None,
update_norm=True)`` and ``update(adv, ret)`` unchanged.

The learner plays plane 0 of every engagement against frozen opponents on plane 1: the pool
(``opp_kind="pool"``: a fixed list of networks with their RunningNorms and sampling weights,
each engagement's opponent redrawn when it autoresets) or one frozen network
(``frozen_opp=(model, norm, holder)``; the MLP keeps no recurrent state, so ``holder`` is unused).
The reference's pool management -- win-rate EMAs, gated snapshots, the league archive,
exploiters and schedules -- is training-loop control outside the rollout/update path and is not
built: ``pool`` is whatever list the caller gives.

collect_rollout returns the reference's (adv, ret, stats): adv and ret (T, nenv), the stats dict
with its keys (ret_sum, len_sum, ep_count, win_sum, loss_sum, alt_loss_sum,
opponent_alt_loss_sum, opponent_ids, win_by_opp, loss_by_opp, ep_by_opp) as device tensors, and
one aggregate finite check (a single host synchronisation) that raises FloatingPointError
before any update, as ppo_gpu.py:2000-2009 does.  adv/ret are the collector's buffers,
overwritten by the next rollout.
"""
from dataclasses import dataclass
from typing import Optional

import torch

from .policy import MLPActorCritic, RunningNorm
from .ppo import LeagueRollout
from .ppo_update import PPOUpdater, UpdateConfig, finite_flag


@dataclass
class PPOGPUConfig:
    """The fields of the reference's PPOGPUConfig (ppo_gpu.py:948-1000) that collection and the
    update read, with the reference's defaults."""
    rollout_steps: int = 32
    gamma: float = 0.997
    gae_lambda: float = 0.95
    clip_coef: float = 0.2
    update_epochs: int = 4
    num_minibatches: int = 8
    lr: float = 3e-4
    critic_lr: Optional[float] = None
    ent_coef: float = 0.0
    vf_coef: float = 0.5
    max_grad_norm: float = 0.5
    target_kl: Optional[float] = 0.03
    normalize_obs: bool = True
    norm_adv: bool = True
    opp_sample: bool = True
    seed: int = 0


class PPOGPUTrainer:
    """env: a GpuDogfightVecEnv.  model: the learner's MLPActorCritic (built from the env's
    observation width when None).  pool: list of (net, RunningNorm or None) frozen opponents;
    None starts it, as the reference does, with the learner itself (its own RunningNorm).
    pool_weights: the opponents' sampling weights (None: uniform)."""

    def __init__(self, env, config=None, model=None, pool=None, pool_weights=None):
        cfg = config if config is not None else PPOGPUConfig()
        if not cfg.normalize_obs:
            raise ValueError("the collectors normalise the learner's observations "
                             "(normalize_obs=True only)")
        self.env, self.cfg, self.nenv = env, cfg, env.nenv
        self.model = (model if model is not None else
                      MLPActorCritic(env.OBS_SIZE).to(env.device))
        self.pool = list(pool) if pool is not None else None
        self.pool_weights = pool_weights
        self.updater = PPOUpdater(self.model, UpdateConfig(
            clip_coef=cfg.clip_coef, update_epochs=cfg.update_epochs,
            num_minibatches=cfg.num_minibatches, lr=cfg.lr, critic_lr=cfg.critic_lr,
            ent_coef=cfg.ent_coef, vf_coef=cfg.vf_coef, max_grad_norm=cfg.max_grad_norm,
            target_kl=cfg.target_kl, norm_adv=cfg.norm_adv), seed=cfg.seed)
        self._collector, self._opp_key = None, None
        self.global_step = 0

    @property
    def norm(self):
        """The learner's RunningNorm (the collector's)."""
        return None if self._collector is None else self._collector.norm

    def _collector_for(self, opp_kind, frozen_opp, update_norm):
        if opp_kind == "pool":
            if self.pool is None:
                # the reference's first pool entry: a frozen copy of the initial learner and of
                # its (initial) RunningNorm
                snap = MLPActorCritic(self.env.OBS_SIZE).to(self.env.device)
                snap.load_state_dict(self.model.state_dict())
                self.pool = [(snap, RunningNorm(self.env.OBS_SIZE, self.env.device))]
            key = ("pool", tuple(id(n) for n, _ in self.pool))
            opps = [n for n, _ in self.pool]
            norms = [m for _, m in self.pool]
            weights = self.pool_weights or [1.0] * len(opps)
        else:
            if frozen_opp is None:
                raise ValueError("opp_kind other than 'pool' needs frozen_opp=(model, norm, "
                                 "holder)")
            key = ("frozen", id(frozen_opp[0]))
            opps, norms, weights = [frozen_opp[0]], [frozen_opp[1]], [1.0]
        if self._collector is None:
            ro = LeagueRollout(self.env, self.model, opps, T=self.cfg.rollout_steps,
                               gamma=self.cfg.gamma, lam=self.cfg.gae_lambda, seed=self.cfg.seed,
                               update_norm=update_norm, opp_weights=weights, opp_norms=norms,
                               stats=True, opp_deterministic=not self.cfg.opp_sample)
            ro.reset()
            self._collector, self._opp_key = ro, key
        elif key != self._opp_key:
            raise ValueError("the opponent set of a trainer is fixed at its first rollout")
        self._collector.update_norm = bool(update_norm)
        return self._collector

    def collect_rollout(self, opp_kind="pool", frozen_opp=None, update_norm=True):
        """One rollout of rollout_steps (ppo_gpu.py:1856-2017); see the module docstring."""
        ro = self._collector_for(opp_kind, frozen_opp, update_norm)
        adv, ret, stats = ro.collect()
        ok = finite_flag((ro.b_obs, ro.b_rew, ro.b_val, ro.b_logp, adv, ret),
                         flags=(ro.finite_acc,))
        if not bool(ok):
            raise FloatingPointError("non-finite physical trajectory or PPO rollout; update refused")
        self.global_step += self.cfg.rollout_steps * self.nenv
        del stats["trajectory_finite"]
        return adv, ret, stats

    def update(self, adv, ret):
        """The PPO update over the last rollout (ppo_gpu.py:2020-2145): PPOUpdater.update's
        result dict (losses, KL, clip fraction, explained variance, grad norms, epochs)."""
        if self._collector is None:
            raise RuntimeError("collect_rollout first")
        return self.updater.update(self._collector, adv, ret)
