"""CPU restatement of the reference's VQ-key decode-attention path.

TEST INFRASTRUCTURE ONLY: importable by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker (or the timed CPU baseline).  The
sunshape_amd package never imports it.  Build the C part with `make -C oracle`.
"""
