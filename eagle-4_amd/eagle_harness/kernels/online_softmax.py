"""The online-softmax step of the verify attention (kernels/online_softmax.py:11-24).

In the reference this is a ``@triton.jit`` helper inlined into each attention kernel. Here the same step (running
row max in the log2 domain, ``alpha = exp2(m_old - m_new)``, ``P = exp2(s - m_new)`` rounded to the value dtype before
``P @ V``, denominator summed in fp32) lives inside the gfx950 attention kernel (``csrc/verify_attention.hip``), on
MFMA score tiles held one query row per lane, so there is nothing to call from Python. :data:`STEP` names the terms
for readers and tests.
"""

STEP = ("row max (log2)", "alpha = exp2(m_old - m_new)", "p = exp2(s - m_new)", "denom = denom * alpha + sum(p)",
        "acc = acc * alpha + p.to(v.dtype) @ v")
