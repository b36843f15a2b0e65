"""CPU oracle for torch_einshard's MI355X path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline.  The product (``torch_einshard``) never imports, links or runs
anything here.

Contents
  einshard_oracle   restatement of the reference's CPU path: its notation ->
                    ``torch.einsum`` equation translation and its pad / unfold
                    / permute chain, run on CPU tensors with the library
                    routines the reference calls (PyTorch is the third-party
                    dependency that holds the arithmetic: torch 2.8.0 pinned by
                    the reference's uv.lock:817-818; this image has 2.10.0).
  brute             plain-C brute force (fp64 einsum by exhaustive loops,
                    closed-form window / halo copy) that pins the restatement.

Pinning status of every oracle function is listed in ``PINNING`` below and
checked by ``tests/test_oracle.py``.
"""

PINNING = {
    "einshard_oracle.equation": "pinned: hand-written equations of reference tests/test_einsum.py:7-87",
    "einshard_oracle.einshard_cpu": (
        "pinned: fp64 brute force (oracle/brute.c) on tiny shapes; closed-form reshape/permute "
        "chains of reference tests/test_einsum.py:90-190; planted-mistake checks"
    ),
    "einshard_oracle.einwindow_cpu": (
        "pinned: known answers of reference tests/test_halo.py:81-96, :123-136, :247-258; "
        "closed-form brute force (oracle/brute.c)"
    ),
    "einshard_oracle.einhalo_cpu": "pinned: known answers of reference tests/test_halo.py:29-50; brute force",
    "einshard_oracle.einconv_cpu": (
        "pinned: the F.conv2d(padding=1) relation of reference tests/test_conv.py:11-78; an fp64 direct sum "
        "over (kernel, channel) on tiny shapes with dilation, asymmetric halos and every boundary"
    ),
    "einshard_oracle.einroll_cpu": (
        "pinned: the explicit index map out[i] = x[(i - s) mod n] on tiny shapes (negative, large and "
        "multiple-of-n shifts); the torch.roll expectation of reference tests/test_distributed_roll.py:10-20"
    ),
}
