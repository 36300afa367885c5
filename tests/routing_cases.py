"""Routing inputs shared by the oracle and GPU tests."""

# Router logits where two exp values differ by one ulp but their
# probabilities round to the same float, with the larger exp value at the
# higher index: ranking by exp value and by probability disagree, and the
# reference's (probability desc, index asc) order must win.
TIE_LOGITS = [
    ([0.012397794052958488, -0.697509229183197, -0.0656374990940094, 0.5141598582267761,
      -0.21968020498752594, -0.16327770054340363, 0.5141599178314209, 0.12348916381597519], (6, 3)),
    ([-0.04776750132441521, 0.16225367784500122, 0.06439773738384247, 0.10661181062459946,
      0.6609346866607666, 0.6609347462654114, 0.23519264161586761, 0.4480293393135071], (5, 4)),
]
