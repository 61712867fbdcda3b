"""Candidate tries: the input format of trie verification (respect/candidates/trie.py)."""
