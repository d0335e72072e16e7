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
                    symmetry, exact round trip.  These fix each CG tensor only
                    up to one sign per cyclic class (l1, l2, l3).  Data pins:
                    the (l,l,0) class (with (0,l,l), (l,0,l)) for l <= 2 by the
                    reference's nablaDFT l = 0 label means, for l = 3 by its
                    OMol on-site f-f means (tests/golden/scale_shifts_*.npz);
                    the 4096-column irreps layout by the OMol scalar columns.
                    The sign of every other class, i.e. every coupling with
                    l1, l2, l3 all > 0 ((1,1,1), (1,1,2), (2,2,2), (1,2,3), ...):
                    parity unpinned.  Only e3nn.o3.wigner_3j, which the
                    reference calls (utils_tensor_decomp.py:93-94) and which is
                    absent here, could pin it; the restatement follows e3nn's
                    published construction.
* matrix2labels.* : exact copy semantics, forward/inverse identity on covered
                    entries.
* irreps_head.*   : node expansion against the CG labels of symmetric on-site
                    blocks, edge pairs against the CG labels of transposed
                    blocks, stable l-sort permutation, SO(3) equivariance.  The
                    e3nn Gate normalisation constants (sigmoid, tanh): parity
                    unpinned (e3nn's own code is absent).
"""
