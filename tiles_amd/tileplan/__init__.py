"""Offline tile planner: package format v10, target description, random-init checkpoints."""
