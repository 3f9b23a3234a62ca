"""The record format the transcript's batch leaves use (reference: setup/)."""
