"""torch_ref -- the canonical attention formula in FP32 torch, the correctness reference.

Plays the role of the reference's ``npu_fa`` backend
(``backends/npu_fa/backend.py:14-49``: ``is_reference=True``, external type,
native GQA) with the arithmetic of the reference's canonical formula
``ref_flash_attn`` (``backends/expert_v2/impl.py:701-716``): key/value heads
repeated per query group, ``softmax(q k^T * scale) v`` in FP32, output rounded
to FP16. It runs on whatever device the canonical tensors live on and walks
the query rows in chunks so an N = 131072 problem never materialises N^2
scores at once.
"""

from fa_amd.harness.contract import Meta

META = Meta(
    name="torch_ref",
    type="external",
    op_type="torch_ref",
    is_reference=True,
    author="fa_amd",
    notes="FP32 softmax(q k^T * scale) v with GQA head mapping, FP16 out; chunked over query rows",
)

# Query rows per chunk: keeps the FP32 score block at <= CHUNK_ELEMS floats.
CHUNK_ELEMS = 1 << 29


def adapt(case, canonical):
    return {
        "q": canonical["q"],
        "k": canonical["k"],
        "v": canonical["v"],
        "heads_q": case.heads_q,
        "scale": case.scale,
    }


def attention(q, k, v, scale, chunk_elems=CHUNK_ELEMS):
    """FP32 ``softmax(q k^T * scale) v`` over [B,H,N,D] tensors, FP16 result."""
    import torch

    b, hq, nq, d = q.shape
    hkv, nk = k.shape[1], k.shape[2]
    if hq % hkv:
        raise ValueError("heads_q must be a multiple of heads_kv")
    group = hq // hkv
    out = torch.empty(q.shape, dtype=torch.float16, device=q.device)
    rows = max(1, min(group * nq, chunk_elems // max(nk, 1)))
    for bi in range(b):
        for hk in range(hkv):
            kf = k[bi, hk].float()
            vf = v[bi, hk].float()
            qg = q[bi, hk * group:(hk + 1) * group].reshape(group * nq, d)
            og = out[bi, hk * group:(hk + 1) * group].view(group * nq, d)
            for r0 in range(0, group * nq, rows):
                s = torch.matmul(qg[r0:r0 + rows].float(), kf.t())
                s.mul_(scale)
                p = torch.softmax(s, dim=-1)
                del s
                og[r0:r0 + rows] = torch.matmul(p, vf).to(torch.float16)
                del p
    return out


def call(op_args):
    return attention(op_args["q"], op_args["k"], op_args["v"], op_args["scale"])
