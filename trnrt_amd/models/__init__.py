"""The DSA selection / slot / attend functions of trnrt/models/dsa_long.py (only those: nothing else of the
reference's model package is mirrored)."""
