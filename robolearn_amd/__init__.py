"""MI355X-native learner hot path for RoboLearn's FlashSAC and PPO updates."""

__version__ = "0.1.0"
