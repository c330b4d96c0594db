"""Paired sine/cosine evaluation for rotary embeddings on the MI355X
(counterpart of the reference's src/sfu_repro/rope/).

Importing this package performs no model or runtime monkey-patching.
"""
