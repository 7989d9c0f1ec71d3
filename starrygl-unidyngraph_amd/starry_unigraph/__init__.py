"""starry_unigraph -- MI355X-native CTDG training step (sampler, memory/mailbox,
time encoding + temporal attention) behind the reference's API."""
__version__ = "0.1.1+mi355x"
