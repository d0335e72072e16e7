"""CPU restatement of CoefficientMapping (reference so3.py:25-133); test oracle only."""
from __future__ import annotations

import torch


class CoefficientMapping:
    def __init__(self, lmax, mmax):
        self.lmax, self.mmax = lmax, mmax
        l_h = torch.tensor([]).long()
        m_h = torch.tensor([]).long()
        m_c = torch.tensor([]).long()
        for l in range(lmax + 1):                      # so3.py:39-44
            mm = min(mmax, l)
            m = torch.arange(-mm, mm + 1).long()
            m_c = torch.cat([m_c, m])
            m_h = torch.cat([m_h, m.abs()])
            l_h = torch.cat([l_h, torch.full_like(m, l)])
        self.l_harmonic, self.m_harmonic, self.m_complex = l_h, m_h, m_c
        n = len(l_h)
        to_m = torch.zeros(n, n)
        self.m_size = [0] * (mmax + 1)
        offset = 0
        idx = torch.arange(n)
        for m in range(mmax + 1):                      # so3.py:52-64
            r = idx[(l_h <= lmax) & (m_c == m)]
            for o, i in enumerate(r):
                to_m[o + offset, i] = 1.0
            offset += len(r)
            self.m_size[m] = len(r)
            if m != 0:
                im = idx[(l_h <= lmax) & (m_c == -m)]
                for o, i in enumerate(im):
                    to_m[o + offset, i] = 1.0
                offset += len(im)
        self.to_m = to_m

    def coefficient_idx(self, lmax, mmax):             # so3.py:126-133
        mask = (self.l_harmonic <= lmax) & (self.m_harmonic <= mmax)
        return torch.arange(len(mask))[mask]
