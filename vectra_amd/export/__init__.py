"""Deployment compile of the price model: bundle export, load and serving."""
