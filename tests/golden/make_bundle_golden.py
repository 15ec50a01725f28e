"""Writes tests/golden/bundle_metadata_golden.json with the reference's own bundle writer
(research/competition_36500/runtime/claude_code/model.py:599-652 save_bundle, called with the
metadata gpu_ckpt_to_bundle.py:165-183 adds) for a 184-D MLPDiscreteActorCritic, and
bundle_norm_golden.npz with the normalisation statistics it was given.  Run in the build
container only (it imports the reference from /root/reference); the outputs are committed."""
import json
import os
import sys
import tempfile

import numpy as np
import torch

REF = "/root/reference/research/competition_36500/runtime"
HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    sys.path.insert(0, REF)
    import re
    import claude_code.model as M
    # the contract string, read from observation_contract.py's text (importing that module pulls
    # in the simulator package, which this path does not need)
    txt = open(os.path.join(REF, "claude_code", "observation_contract.py"), encoding="utf-8").read()
    CUDA_OBSERVATION_CONTRACT = re.search(r'CUDA_OBSERVATION_CONTRACT = "([^"]+)"', txt).group(1)
    torch.manual_seed(0)
    model = M.make_actor_critic(obs_dim=184, act_dim=4, num_bins=21, hidden=(256, 256),
                                activation="tanh")
    rng = np.random.default_rng(0)
    mean = rng.normal(0, 1, 184)
    var = rng.uniform(0.5, 2.0, 184)
    obs_norm = {"mean": mean.tolist(), "var": var.tolist(), "count": 12345.0}
    extra = {"reward_module": "claude_code.my_reward",
             "observation_module": "claude_code.my_observation",
             "observation_mode": "claude164r", "selected_iteration": 7,
             "source": "gpu_ckpt_to_bundle:golden.pt", "trainer": "cuda_fdm.PPOGPUTrainer",
             "observation_contract": CUDA_OBSERVATION_CONTRACT, "policy_hz": 10,
             "action_repeat": 6, "training_protocol": "golden_protocol",
             "auxiliary_trained": False, "auxiliary_contract": None}
    with tempfile.TemporaryDirectory() as d:
        M.save_bundle(model, d, obs_norm=obs_norm, extra_metadata=extra)
        meta = json.loads(open(os.path.join(d, M.METADATA_FILENAME), encoding="utf-8").read())
    with open(os.path.join(HERE, "bundle_metadata_golden.json"), "w", encoding="utf-8") as fh:
        json.dump(meta, fh, indent=2, ensure_ascii=False)
    np.savez(os.path.join(HERE, "bundle_norm_golden.npz"), mean=mean, var=var,
             count=np.array(12345.0))
    print("wrote", sorted(meta))


if __name__ == "__main__":
    main()
