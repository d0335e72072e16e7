"""CPU oracle for the MALOQ equivariant message-passing hot path.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU, the algorithms of
the reference's pure-PyTorch / NumPy backends (each function cites the
reference file:line it follows).  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it, and only as the checker
or the reported CPU baseline: it is never the measured or shipped path, and
the product (``maloq_amd``) never imports it.

Parity pins (what each restated function is checked against):
* rotation.*      : reference Jd.pt values (tests/golden/jd_reference.npz),
                    D D^T = I, homomorphism, edge-frame alignment D^1 v = |v| e_y.
* so3.*           : closed-form ordering rules, exact integer tables.
* so2.*, message.*: brute force on tiny inputs, gamma invariance of the block,
                    global SO(3) equivariance, fp64 scatter sums.
* tensor_decomp.* : CG invariance under the Jd-based D, unit norm, cyclic
                    symmetry, exact round trip, (0,l,l)/(l,l,0) sign pinned by the
                    reference's element_scale_shifts data (l=0 label means).
                    Sign of CG tensors with l1+l2+l3 odd: parity unpinned (only
                    an import of e3nn could pin it; e3nn is absent).
* matrix2labels.* : exact copy semantics, forward/inverse identity on covered
                    entries.
* irreps_head.*   : node expansion against the CG labels of symmetric on-site
                    blocks, edge pairs against the CG labels of transposed
                    blocks, stable l-sort permutation, SO(3) equivariance.  The
                    e3nn Gate normalisation constants (sigmoid, tanh): parity
                    unpinned (e3nn's own code is absent).
"""
