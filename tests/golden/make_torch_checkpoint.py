"""Write a small FlashSAC checkpoint directory in the reference's Torch format.

Runs only where the reference tree is mounted (this build container); tests
read the committed files under tests/golden/torch_checkpoint/.  The network
files are written by the reference's own Network.save
(robolearn/flashsac/_utils/network.py:115-127) and RewardNormalizer.save
(robolearn/flashsac/_utils/reward_normalization.py:136-151), after two Adam +
LambdaLR steps on seeded gradients, so they hold real optimizer and scheduler
state.  agent_state.pt and config.json are the two small dicts
robolearn/flashsac/agent.py:529-551 writes beside them (agent.py itself needs
gymnasium, which the image lacks, so those two are composed here the same way).

Imports only torch/numpy modules of the reference: flashsac/config.py,
networks.py, _utils/network.py, _utils/scheduler.py,
_utils/reward_normalization.py.

Usage: python tests/golden/make_torch_checkpoint.py [reference_src]
"""

import json
import sys
from dataclasses import asdict
from pathlib import Path

import torch

OUT = Path(__file__).resolve().parent / "torch_checkpoint"

# Dimensions and config of the fixture; tests build the MI355X agent with the same values.
OBS, ACT, ENVS = 4, 2, 3
CONFIG = dict(device="cpu", seed=0, actor_num_blocks=1, actor_hidden_dim=16, critic_num_blocks=2,
              critic_hidden_dim=16, critic_num_bins=11, critic_min_v=-10.0, critic_max_v=10.0,
              learning_rate_init=1e-4, learning_rate_peak=3e-4, learning_rate_end=1e-4, learning_rate_warmup_step=1,
              learning_rate_decay_step=50, buffer_max_length=64, buffer_min_length=8, sample_batch_size=8)


def main(src: str) -> None:
    sys.dont_write_bytecode = True  # the reference tree is read-only input: leave no __pycache__ in it
    sys.path.insert(0, src)
    from robolearn.flashsac._utils.network import Network
    from robolearn.flashsac._utils.reward_normalization import RewardNormalizer
    from robolearn.flashsac._utils.scheduler import warmup_cosine_decay_scheduler
    from robolearn.flashsac.config import FlashSACConfig
    from robolearn.flashsac.networks import FlashSACActor, FlashSACDoubleCritic, FlashSACTemperature

    torch.set_num_threads(1)
    cfg = FlashSACConfig(**CONFIG)
    schedule = warmup_cosine_decay_scheduler(cfg.learning_rate_init, cfg.learning_rate_peak, cfg.learning_rate_end,
                                             cfg.learning_rate_warmup_step, cfg.learning_rate_decay_step)
    g = torch.Generator().manual_seed(77)

    def trained(module, weight_normalization, steps=2):
        optimizer = torch.optim.Adam(module.parameters(), lr=cfg.learning_rate_peak)
        scheduler = torch.optim.lr_scheduler.LambdaLR(
            optimizer, lr_lambda=lambda step: schedule(step) / cfg.learning_rate_peak)
        net = Network(network=module, optimizer=optimizer, scheduler=scheduler,
                      use_weight_normalization=weight_normalization)
        project = net.normalize_parameters if weight_normalization else (lambda: None)
        project()
        for _ in range(steps):
            for p in module.parameters():
                p.grad = torch.randn(p.shape, generator=g) * 0.1
            optimizer.step()
            scheduler.step()
            project()
        with torch.no_grad():  # non-trivial BatchNorm running statistics
            for name, buffer in module.named_buffers():
                if name.endswith("running_mean"):
                    buffer.copy_(torch.randn(buffer.shape, generator=g) * 0.2)
                elif name.endswith("running_var"):
                    buffer.copy_(torch.rand(buffer.shape, generator=g) + 0.5)
        return net

    torch.manual_seed(0)
    actor = trained(FlashSACActor(num_blocks=cfg.actor_num_blocks, input_dim=OBS, hidden_dim=cfg.actor_hidden_dim,
                                  action_dim=ACT), True)
    critic_module = FlashSACDoubleCritic(num_blocks=cfg.critic_num_blocks, input_dim=OBS + ACT,
                                         hidden_dim=cfg.critic_hidden_dim, num_bins=cfg.critic_num_bins,
                                         min_v=cfg.critic_min_v, max_v=cfg.critic_max_v)
    critic = trained(critic_module, True)
    target_module = FlashSACDoubleCritic(num_blocks=cfg.critic_num_blocks, input_dim=OBS + ACT,
                                         hidden_dim=cfg.critic_hidden_dim, num_bins=cfg.critic_num_bins,
                                         min_v=cfg.critic_min_v, max_v=cfg.critic_max_v)
    target_module.load_state_dict(critic_module.state_dict())
    with torch.no_grad():
        for p in target_module.parameters():
            p.add_(torch.randn(p.shape, generator=g) * 0.01)
    target = Network(network=target_module, use_weight_normalization=True)
    temperature = trained(FlashSACTemperature(cfg.temp_initial_value), False)

    normalizer = RewardNormalizer(gamma=cfg.gamma, G_max=cfg.normalized_G_max, load_rms=True,
                                  device=torch.device("cpu"))
    for _ in range(4):
        normalizer.update_reward_stats(reward=torch.randn(ENVS, generator=g),
                                       terminated=torch.rand(ENVS, generator=g) < 0.3,
                                       truncated=torch.zeros(ENVS, dtype=torch.bool))

    OUT.mkdir(parents=True, exist_ok=True)
    metadata = {"observation_dim": OBS, "critic_observation_dim": None, "action_dim": ACT, "config": asdict(cfg)}
    with open(OUT / "config.json", "w") as stream:
        json.dump(metadata, stream, indent=2)
        stream.write("\n")
    actor.save(str(OUT / "actor.pt"))
    critic.save(str(OUT / "critic.pt"))
    target.save(str(OUT / "target_critic.pt"))
    temperature.save(str(OUT / "temperature.pt"))
    normalizer.save(str(OUT / "reward_normalizer.pt"))
    torch.save({"update_step": 4, "grad_scaler_state_dict": {}}, OUT / "agent_state.pt")
    sizes = {p.name: p.stat().st_size for p in sorted(OUT.iterdir())}
    print(f"wrote {OUT}: {sizes}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
