"""TEST INFRASTRUCTURE ONLY -- the CPU oracle of the fused linear + CE path.

Nothing in the product (mini_trainer_amd/, include/, the built library)
imports, links or runs anything in this directory.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
checker (and as the timed CPU baseline), never as the thing measured.

Contents
  torch_path.py  the reference's own arithmetic on the CPU: F.linear in the
                 input dtype -> .float() -> [softcap] -> F.cross_entropy(
                 reduction='none', ignore_index) and its autograd backward
                 (none_reduction_losses.py:35, TF/loss/loss_utils.py:59,
                 train.py:97-104), chunked over rows; dW accumulated in fp32.
  brute.py       float64 closed forms on tiny shapes (pins torch_path and
                 the C restatement).
  flce_ref.c     plain-C restatement of the fused algorithm (valid-row
                 compaction, tiled online log-sum-exp, G / dX / dW, segment
                 sums, materialised-logits CE) with double accumulation;
                 built by build.py into oracle/_build/, loaded by ref.py.
Pinning of every function is listed in the headers of those files.
"""
