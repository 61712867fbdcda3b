"""Verification-step host code: the decoder forward over the C-ABI kernels,
trie verification, greedy acceptance, KV compaction and the token-by-token
reference path (mirrors respect/decoding)."""
