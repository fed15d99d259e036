"""GPU tests of the greedy tokens handed from one forward to the next as the
lm_head's argmax keys (no reduction launch in between):

* nsg_lm_head_fold_keys + nsg_embed_rows_keys: the key column of the ids
  receives exactly the tokens nsg_lm_head_fold_argmax writes, the other ids
  stay, and every row is the embedding of its (new) id, with the partial sums
  of squares of those rows;
* nsg_spec_accept_greedy_keys: the outputs, rollback slots and target tokens
  of nsg_spec_accept_greedy_tokens on those tokens, for accepted prefixes of
  every length;
* the engine's captured greedy step uses the keys and emits the tokens of
  the eager step (which reduces them with its own launch)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _rand(shape, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(*shape, generator=g, device="cuda") * scale).bfloat16()


def _head(M, N, seed, K=896):
    from nanosglang_amd import kernels
    x = _rand((M, K), seed=seed, scale=2.0)
    w = _rand((N, K), seed=seed + 1, scale=K ** -0.5)
    return x, w, kernels.row_sumsq(x)


@pytest.mark.parametrize("B,J,key_j,N", [(32, 1, 0, 151936), (7, 1, 0, 1000), (32, 5, 4, 151936),
                                         (3, 5, 2, 1000)])
def test_embed_rows_takes_the_key_column(B, J, key_j, N):
    from nanosglang_amd import kernels
    print(f"case: embed keys B={B} J={J} key_j={key_j} N={N}", flush=True)
    x, w, ss = _head(B, N, seed=B * 10 + J)
    lib = kernels._lib()
    keys = torch.zeros(lib.nsg_linear_argmax_workspace_bytes(B, N) // 8, dtype=torch.int64,
                       device="cuda")
    kc = kernels.lm_head_fold(x, w, ss, EPS, keys_out=keys)
    tok = kernels.lm_head_fold(x, w, ss, EPS,
                               argmax_out=torch.empty(B, dtype=torch.int64, device="cuda"))
    # ids: the verify layout, position-major (J, B) storage seen as (B, J)
    g = torch.Generator(device="cuda").manual_seed(B + J)
    ids_pm = torch.randint(0, N, (J, B), generator=g, device="cuda")
    before = ids_pm.clone()
    ids = ids_pm.t() if J > 1 else ids_pm[0]
    table = _rand((N, 896), seed=77)
    ssq = torch.full((896 // 16, B * J), -1.0, device="cuda")
    out = kernels.embed_rows(ids, table, sumsq_out=ssq, keys=(keys, kc, key_j))
    torch.cuda.synchronize()
    assert 1 <= kc <= 4 * ((N + 127) // 128)
    expect = before.clone()
    expect[key_j] = tok
    assert torch.equal(ids_pm, expect)
    ref = torch.nn.functional.embedding((expect.t() if J > 1 else expect[0]).reshape(-1), table)
    assert torch.equal(out, ref)
    assert torch.equal(ssq, kernels.row_sumsq(ref))


@pytest.mark.parametrize("B,k", [(1, 4), (32, 4), (7, 8)])
def test_accept_greedy_keys_equals_tokens(B, k):
    from nanosglang_amd import kernels
    print(f"case: accept greedy keys B={B} k={k}", flush=True)
    N, P = 151936, 16
    M = B * (k + 1)
    x, w, ss = _head(M, N, seed=M)
    lib = kernels._lib()
    keys = torch.empty(lib.nsg_linear_argmax_workspace_bytes(M, N) // 8, dtype=torch.int64,
                       device="cuda")
    kc = kernels.lm_head_fold(x, w, ss, EPS, keys_out=keys)
    ttok = kernels.lm_head_fold(x, w, ss, EPS,
                                argmax_out=torch.empty(M, dtype=torch.int64, device="cuda"))
    t2 = ttok.view(B, k + 1)
    # drafts agreeing with the target on a prefix of every length
    rng = np.random.default_rng(B + k)
    drafts = torch.randint(0, N, (B, k), device="cuda")
    for b in range(B):
        a = int(rng.integers(0, k + 1))
        drafts[b, :a] = t2[b, :a]
    # a position-major id buffer's columns as the draft view (any strides)
    ids_pm = torch.zeros(k + 1, B, dtype=torch.int64, device="cuda")
    ids_pm[1:] = drafts.t()
    dview = ids_pm.t()[:, 1:]
    start = torch.tensor(rng.integers(20, 200, B), dtype=torch.int32, device="cuda")
    npg = ((start.cpu().numpy() + k + 1 + P - 1) // P).astype(np.int32)
    kvp = torch.tensor(np.concatenate([[0], np.cumsum(npg)]), dtype=torch.int32, device="cuda")
    idx = torch.tensor(rng.permutation(4000)[:int(npg.sum())], dtype=torch.int32, device="cuda")
    ref = kernels.spec_accept_greedy_tokens(t2.contiguous(), dview, N, kvp, idx, start,
                                            page_size=P)
    tout = torch.full((M,), -7, dtype=torch.int64, device="cuda")
    got = kernels.spec_accept_greedy_keys(keys, kc, B, k, dview, N, kvp, idx, start,
                                          page_size=P, target_tokens_out=tout)
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    assert torch.equal(tout, ttok)


def test_engine_graph_step_hands_tokens_on_as_keys():
    """The captured greedy step (keys mode) emits the eager step's tokens."""
    from nanosglang_amd.engine.spec_engine import SpecEngine
    from nanosglang_amd.model.causal_lm import CausalLM, ModelConfig
    from oracle.model import ModelConfig as OCfg, init_weights
    print("case: engine keys mode, graph vs eager", flush=True)
    tiny = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=4,
                num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024)
    wts = init_weights(OCfg(**tiny), seed=3)
    for L in wts["layers"]:
        for key in ("q", "k", "v", "o", "gate", "up", "down"):
            L[key] *= 8.0
    model = CausalLM(ModelConfig(**tiny), weights=wts)
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, 1000, n).tolist() for n in (20, 33, 5, 64, 12)]
    outs = []
    for graphs in (True, False):
        eng = SpecEngine(model, draft_layers=2, num_speculative=4, num_blocks=128, max_batch=8,
                         use_graphs=graphs)
        if graphs:
            assert eng._keys_mode(8) and eng._keys_mode(1)
        outs.append(eng.generate(prompts, [24, 9, 30, 17, 21]))
        eng.check_device_flags()
    assert outs[0] == outs[1]
