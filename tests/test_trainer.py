"""PPOGPUTrainer's entry points (trainer.py; research/competition_36500/runtime/cuda_fdm/
ppo_gpu.py:1856-2145): collect_rollout's episode and match bookkeeping and its refusal of a
non-finite trajectory, against hand-counted cases on the CPU and the rollout's own buffers on
the GPU."""
from types import SimpleNamespace

import pytest
import torch

from conftest import import_pkg

STAT_KEYS = {"ret_sum", "len_sum", "ep_count", "win_sum", "loss_sum", "alt_loss_sum",
             "opponent_alt_loss_sum", "opponent_ids", "win_by_opp", "loss_by_opp", "ep_by_opp"}


def _book(nenv, nopp, min_alt=304.8):
    """A stand-in collector holding what LeagueRollout._stats_step reads (CPU tensors)."""
    z = lambda: torch.zeros((), dtype=torch.float32)
    o = SimpleNamespace(nenv=nenv, min_alt=min_alt,
                        ep_ret=torch.zeros(nenv), ep_len=torch.zeros(nenv),
                        _thp=torch.zeros(2 * nenv, dtype=torch.float64),
                        _talt=torch.zeros(2 * nenv, dtype=torch.float64))
    st = {"ret_sum": z(), "len_sum": z(), "ep_count": z(), "win_sum": z(), "loss_sum": z(),
          "alt_loss_sum": z(), "opponent_alt_loss_sum": z(),
          "opponent_ids": torch.arange(nopp), "win_by_opp": torch.zeros(nopp),
          "loss_by_opp": torch.zeros(nopp), "ep_by_opp": torch.zeros(nopp)}
    return o, st


def test_match_bookkeeping_known_cases():
    """Seven engagements ending (or not) in the outcomes ppo_gpu.py:1950-1969 distinguishes:
    0 learner shot down -> loss; 1 opponent shot down -> win; 2 learner below the deck -> loss
    and an altitude loss; 3 opponent below the deck -> win and an opponent altitude loss;
    4 both alive, learner ahead on HP -> win; 5 both alive, equal HP -> draw; 6 not done."""
    P = import_pkg("ppo")
    o, st = _book(7, 3)
    hp = [(0.0, 1.0), (1.0, 0.0), (1.0, 1.0), (1.0, 1.0), (0.9, 0.5), (0.7, 0.7), (0.0, 1.0)]
    alt = [(5000, 5000), (5000, 5000), (200, 5000), (5000, 100), (5000, 5000), (5000, 5000),
           (5000, 5000)]
    o._thp.copy_(torch.tensor([x for p in hp for x in p], dtype=torch.float64))
    o._talt.copy_(torch.tensor([x for p in alt for x in p], dtype=torch.float64))
    done = torch.tensor([1, 1, 1, 1, 1, 1, 0], dtype=torch.float32)
    rew = torch.tensor([1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0])
    assign = torch.tensor([0, 1, 2, 0, 1, 2, 0], dtype=torch.int32)
    o.ep_ret.fill_(0.5)
    o.ep_len.fill_(9.0)
    P.LeagueRollout._stats_step(o, st, rew, done, assign)
    assert float(st["win_sum"]) == 3.0 and float(st["loss_sum"]) == 2.0
    assert float(st["alt_loss_sum"]) == 1.0 and float(st["opponent_alt_loss_sum"]) == 1.0
    assert float(st["ep_count"]) == 6.0
    assert float(st["ret_sum"]) == pytest.approx(sum(0.5 + r for r in (1, 2, 3, 4, 5, 6)))
    assert float(st["len_sum"]) == 6 * 10.0
    assert st["win_by_opp"].tolist() == [1.0, 2.0, 0.0]          # engagements 3; 1, 4
    assert st["loss_by_opp"].tolist() == [1.0, 0.0, 1.0]         # engagements 0, 2
    assert st["ep_by_opp"].tolist() == [2.0, 2.0, 2.0]
    # finished engagements restart their running return and length; the live one keeps them
    assert o.ep_ret.tolist() == [0.0] * 6 + [7.5] and o.ep_len.tolist() == [0.0] * 6 + [10.0]


def test_trainer_config_defaults_follow_the_reference():
    T = import_pkg("trainer")
    c = T.PPOGPUConfig()
    assert (c.rollout_steps, c.gamma, c.gae_lambda, c.clip_coef, c.update_epochs,
            c.num_minibatches, c.lr, c.vf_coef, c.max_grad_norm, c.target_kl) == \
        (32, 0.997, 0.95, 0.2, 4, 8, 3e-4, 0.5, 0.5, 0.03)


def _env(nenv, seed):
    E = import_pkg("rl_env").GpuDogfightVecEnv
    return E(nenv, seed=seed, max_engage_time_s=4.0, ic_pool_size=256)


@pytest.mark.gpu
def test_collect_rollout_pool_and_update(gpu):
    """collect_rollout(opp_kind="pool") with the default pool (a frozen copy of the learner):
    the reference's stats keys; completed episodes equal the done flags the rollout wrote;
    returns and lengths equal a host recount of the rewards and flags; the per-opponent counts
    sum to the totals; then update(adv, ret) runs on the same buffers."""
    T = import_pkg("trainer")
    env = _env(256, 3)
    tr = T.PPOGPUTrainer(env, T.PPOGPUConfig(rollout_steps=48, seed=5))
    adv, ret, st = tr.collect_rollout()
    assert set(st) == STAT_KEYS
    assert adv.shape == (48, 256) and ret.shape == (48, 256)
    ro = tr._collector
    done = torch.cat([ro.b_done[1:], ro.next_done[None]]).cpu()      # done after step t
    rew = ro.b_rew.cpu()
    assert float(st["ep_count"]) == float(done.sum()) > 0
    ep_ret = torch.zeros(256)
    ep_len = torch.zeros(256)
    rs, ls = 0.0, 0.0
    for t in range(48):
        ep_ret += rew[t]
        ep_len += 1.0
        rs += float((ep_ret * done[t]).sum())
        ls += float((ep_len * done[t]).sum())
        ep_ret *= 1.0 - done[t]
        ep_len *= 1.0 - done[t]
    assert float(st["ret_sum"]) == pytest.approx(rs, rel=1e-5, abs=1e-3)
    assert float(st["len_sum"]) == ls
    assert float(st["win_by_opp"].sum()) == float(st["win_sum"])
    assert float(st["loss_by_opp"].sum()) == float(st["loss_sum"])
    assert float(st["ep_by_opp"].sum()) == float(st["ep_count"])
    assert float(st["win_sum"]) + float(st["loss_sum"]) <= float(st["ep_count"])
    assert tr.global_step == 48 * 256
    res = tr.update(adv, ret)
    assert res["optimizer_steps"] >= 8 and bool(torch.isfinite(res["pl"]))
    adv2, ret2, st2 = tr.collect_rollout(update_norm=False)       # the same collector again
    assert set(st2) == STAT_KEYS and bool(torch.isfinite(adv2).all())
    with pytest.raises(ValueError):
        tr.collect_rollout(opp_kind="frozen", frozen_opp=(tr.model, None, {}))


@pytest.mark.gpu
def test_collect_rollout_frozen_and_nonfinite_refusal(gpu):
    """opp_kind="frozen" plays one frozen network without normalisation (norm None, as the
    reference passes raw observations then) with argmax actions when opp_sample is False; a NaN
    planted in one aircraft's state makes collect_rollout raise FloatingPointError."""
    T = import_pkg("trainer")
    pol = import_pkg("policy")
    env = _env(128, 4)
    opp = pol.MLPActorCritic(184, generator=torch.Generator().manual_seed(9)).to(gpu)
    tr = T.PPOGPUTrainer(env, T.PPOGPUConfig(rollout_steps=16, opp_sample=False))
    frozen = (opp, None, {})
    adv, ret, st = tr.collect_rollout(opp_kind="frozen", frozen_opp=frozen)
    assert set(st) == STAT_KEYS and st["ep_by_opp"].numel() == 1
    assert tr._collector.opp_deterministic
    env.sim.states[17, 5] = float("nan")
    with pytest.raises(FloatingPointError):
        tr.collect_rollout(opp_kind="frozen", frozen_opp=frozen)
