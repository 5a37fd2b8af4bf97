"""The price Transformer whose spatial-attention sites the `vectra` backend
rewrites (the reference's models/price_transformer)."""
