"""Seeded synthetic paged-attention batches shared by the CPU and GPU tests."""
import numpy as np


def make_batch(seed, q_lens, kv_lens, Hq, Hkv, D, P=16, num_pages=None, kv_scale=0.5,
               dtype=np.float32):
    """Pages of every request drawn as a random permutation of the pool, which
    is filled with noise.  Returns a dict of numpy arrays (values are exactly
    representable in bf16 when ``dtype`` is float32)."""
    rng = np.random.default_rng(seed)
    B = len(q_lens)
    need = [(L + P - 1) // P for L in kv_lens]
    if num_pages is None:
        num_pages = sum(need) + 7
    perm = rng.permutation(num_pages)
    tables, off = [], 0
    for n in need:
        tables.append(perm[off:off + n].tolist())
        off += n
    qo = np.zeros(B + 1, np.int32)
    qo[1:] = np.cumsum(q_lens)
    kv_indptr = np.zeros(B + 1, np.int32)
    kv_indptr[1:] = np.cumsum(need)
    kv_indices = np.asarray(sum(tables, []), np.int32)
    last = np.asarray([(L % P) or P for L in kv_lens], np.int32)

    def bf(x):
        import torch
        return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).float().numpy()

    q = bf(rng.standard_normal((int(qo[-1]), Hq, D)))
    k = bf(kv_scale * rng.standard_normal((num_pages, P, Hkv, D)))
    v = bf(kv_scale * rng.standard_normal((num_pages, P, Hkv, D)))
    return dict(q=q, k=k, v=v, qo_indptr=qo, kv_indptr=kv_indptr, kv_indices=kv_indices,
                kv_last_page_len=last, tables=tables)
