"""The serving path that feeds the compiled price model: dynamic batching
(batcher), pinned multi-slot host-to-device staging (feeder) and batched
prediction (predict)."""
