"""Leaf encoding, BLAKE3 leaf hashing and the RFC 6962 Merkle tree, on the GPU."""
