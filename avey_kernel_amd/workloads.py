"""Seeded synthetic inputs for the five benchmark configurations, plus their
algorithmic work (useful flops) and compulsory HBM bytes.

Configurations (C1 is the reference's CPU-sized case, C2 the headline):

====  ======  =====  ====  ===  =====  ==========================================
tag   op      dtype  B     N    D      notes
====  ======  =====  ====  ===  =====  ==========================================
C1    avey    fp32   2     64   64     x [2,64,128] split: z_tl = x[..., :64],
                                       z_tr = x[..., 64:]; seed 0
C2    avey    bf16   16    256  768    causal, gate ~ N(0,1); seed 1
C3    avey_b  bf16   32    512  768    bidirectional, full tiles; seed 2
C4    avey    bf16   4     2048 1024   causal; 1% of rows x50; seed 3
C5    avey_b  bf16   256   128  512    key padding, L_b ~ U[64,128]; seed 4
====  ======  =====  ====  ===  =====  ==========================================

Every config draws, in this order from one CPU generator: x ~ N(0,1) [B,N,Dx],
the gate ~ N(0,1) [B,N,D] (not for C1, whose gate is the left half of x), and V
~ U(-1/sqrt(N), 1/sqrt(N)) [N,N] as an fp32 master; then the config's extra
draws (C4: row indices to scale, C5: valid lengths). Bias is zeros. Casting to
the config dtype happens last (round to nearest even). For the Avey-B configs V
is drawn to fix the random stream but only the ``avey(..., causal=False)``
variant uses it.

Useful flops F = 4 * D * sum_b P_b, where P_b is the number of allowed
(query, key) pairs (causal N(N+1)/2, bidirectional N^2, padded L_b^2): 2 for
each similarity dot product and 2 for each mixing multiply-add. Compulsory
bytes M = z_tr + z_tl + out (+ V if used, + bias, + valid).
"""

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Config:
    tag: str
    op: str          # 'avey' or 'avey_b'
    dtype: torch.dtype
    batch: int
    context: int
    features: int
    seed: int
    causal: bool

    @property
    def name(self):
        return (f'{self.tag}:{self.op}{"-causal" if self.causal else ""}-'
                f'{str(self.dtype).replace("torch.", "")}-B{self.batch}-N{self.context}-D{self.features}')


CONFIGS = {
    'C1': Config('C1', 'avey', torch.float32, 2, 64, 64, 0, True),
    'C2': Config('C2', 'avey', torch.bfloat16, 16, 256, 768, 1, True),
    'C3': Config('C3', 'avey_b', torch.bfloat16, 32, 512, 768, 2, False),
    'C4': Config('C4', 'avey', torch.bfloat16, 4, 2048, 1024, 3, True),
    'C5': Config('C5', 'avey_b', torch.bfloat16, 256, 128, 512, 4, False),
}
HEADLINE = 'C2'


def make_inputs(cfg, device='cpu', dtype=None):
    """Deterministic inputs for a config: dict(z_tr, z_tl, v, bias, valid)."""
    dtype = dtype or cfg.dtype
    g = torch.Generator(device='cpu').manual_seed(cfg.seed)
    b, n, d = cfg.batch, cfg.context, cfg.features
    if cfg.tag == 'C1':
        x = torch.randn(b, n, 2 * d, generator=g)
        z_tl, z_tr = x[..., :d].contiguous(), x[..., d:].contiguous()
    else:
        z_tr = torch.randn(b, n, d, generator=g)
        z_tl = torch.randn(b, n, d, generator=g)
    v = (torch.rand(n, n, generator=g) * 2 - 1) / math.sqrt(n)
    valid = None
    if cfg.tag == 'C4':
        rows = torch.randperm(b * n, generator=g)[:math.ceil(0.01 * b * n)]
        z_tr.view(-1, d)[rows] *= 50
    if cfg.tag == 'C5':
        lengths = torch.randint(64, n + 1, (b,), generator=g)
        valid = torch.arange(n)[None, :] < lengths[:, None]
        z_tr[~valid] = 0
        z_tl[~valid] = 0
    bias = torch.zeros(d)
    out = {'z_tr': z_tr.to(dtype), 'z_tl': z_tl.to(dtype), 'v': v.to(dtype), 'bias': bias.to(dtype),
           'valid': valid}
    return {k: (t.to(device) if t is not None else None) for k, t in out.items()}


def allowed_pairs(cfg, valid=None):
    """Number of (query, key) pairs that contribute, summed over the batch."""
    n = cfg.context
    if valid is not None:
        lengths = valid.sum(dim=1).to(torch.int64)
        if cfg.causal:
            return int((lengths * (lengths + 1) // 2).sum())
        return int((lengths * lengths).sum())
    per = n * (n + 1) // 2 if cfg.causal else n * n
    return cfg.batch * per


def useful_flops(cfg, valid=None):
    return 4 * cfg.features * allowed_pairs(cfg, valid)


def dense_flops(cfg):
    """Dense-equivalent flops: every (query, key) pair, as the eager path computes them
    (two dense B x C x C x D products, ops.py:69,78). Reported only as such."""
    return 4 * cfg.features * cfg.batch * cfg.context * cfg.context


def compulsory_bytes(cfg, with_v=None):
    es = torch.finfo(cfg.dtype).bits // 8
    with_v = (cfg.op == 'avey') if with_v is None else with_v
    act = cfg.batch * cfg.context * cfg.features * es
    total = 3 * act + cfg.features * es  # z_tr, z_tl, out, bias
    if with_v:
        total += cfg.context * cfg.context * es
    if cfg.tag == 'C5':
        total += cfg.batch * cfg.context  # valid bytes
    return total


def call(cfg, inputs, backend='auto', activation='identity'):
    """Run the config's public op (``avey`` or ``avey_b``) on prepared inputs."""
    from .ops import avey, avey_b
    if cfg.op == 'avey':
        return avey(inputs['z_tr'], inputs['v'], z_tl=inputs['z_tl'], bias=inputs['bias'],
                    valid=inputs['valid'], causal=cfg.causal, activation=activation, backend=backend)
    return avey_b(inputs['z_tr'], z_tl=inputs['z_tl'], bias=inputs['bias'], valid=inputs['valid'],
                  activation=activation, backend=backend)
