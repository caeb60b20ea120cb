"""Benchmark inputs: seeded synthetic decode steps for the BASELINE.json configurations
(:mod:`amass.bench.synth`).  Timing and the JSON report live in the repository's bench.py."""
