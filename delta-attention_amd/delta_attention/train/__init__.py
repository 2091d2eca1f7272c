"""Training path of delta attention: the differentiable layer
(delta_attention/train/flex_delta.py)."""
