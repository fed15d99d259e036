"""The pipelined decode loop of SpecEngine.generate (graph mode) and the host
gate under it:
* nsg_host_gate_wait holds the stream until the host raises the flag, then
  copies the pinned staging bytes the host wrote before raising it, resets
  the flag, and gives up after its timeout with bit 0 of the error word set
  (the timeout forced from the host: the flag is never raised);
* pipelined generate emits exactly the tokens of the unpipelined loop, greedy
  and stochastic, with requests finishing at different steps, returns every
  page, and leaves no error flag;
* an exception between queueing a step and releasing it releases the held
  step and leaves the engine usable."""
import ctypes as C
import time

import numpy as np
import pytest
import torch

from nanosglang_amd import _native

pytestmark = pytest.mark.gpu

TINY = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=4,
            num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024)


def _model():
    from nanosglang_amd.model.causal_lm import CausalLM, ModelConfig
    from oracle.model import ModelConfig as OCfg, init_weights
    w = init_weights(OCfg(**TINY), seed=3)
    for L in w["layers"]:
        for key in ("q", "k", "v", "o", "gate", "up", "down"):
            L[key] *= 8.0
    return CausalLM(ModelConfig(**TINY), weights=w)


def test_host_gate_releases_on_flag_and_gives_up_after_timeout():
    lib = _native.load()
    print("case: host gate release and timeout", flush=True)
    p = C.c_void_p()
    _native.check(lib.nsg_host_gate_alloc(C.byref(p)), "nsg_host_gate_alloc")
    flag = C.c_int32.from_address(p.value)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    src = torch.zeros(40_000, dtype=torch.uint8, pin_memory=True)   # 2500 x 16 bytes
    dst = torch.zeros(40_000, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def gate(timeout_us, n):
        return lib.nsg_host_gate_wait(p.value, err.data_ptr(), timeout_us, src.data_ptr(),
                                      dst.data_ptr(), n, stream)
    try:
        assert flag.value == 0
        # held until the flag is raised: the fill queued behind it has not
        # run, and the copy takes what the host wrote before raising it
        _native.check(gate(5_000_000, 40_000), "nsg_host_gate_wait")
        out.fill_(7)
        time.sleep(0.05)
        assert not torch.cuda.current_stream().query()
        data = torch.randint(0, 256, (40_000,), dtype=torch.uint8)
        src.copy_(data)
        flag.value = 1
        torch.cuda.synchronize()
        assert int(out.item()) == 7 and int(err.item()) == 0
        assert torch.equal(dst.cpu(), data)
        assert flag.value == 0                      # the gate reset it
        # never raised: gives up after 20 ms, error bit 0, flag still 0
        t0 = time.perf_counter()
        _native.check(gate(20_000, 0), "nsg_host_gate_wait")
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        print(f"  timeout path returned after {dt * 1e3:.1f} ms", flush=True)
        assert int(err.item()) == 1 and flag.value == 0
        assert 0.015 < dt < 2.0
        # argument checks: no launch
        assert gate(0, 0) == 1
        assert gate(1000, 24) == 1                  # not a multiple of 16
        assert lib.nsg_host_gate_wait(None, err.data_ptr(), 1000, None, None, 0, stream) == 1
    finally:
        torch.cuda.synchronize()
        _native.check(lib.nsg_host_gate_free(p.value), "nsg_host_gate_free")


def test_host_gate_segments_copy_only_their_ranges():
    """nsg_host_gate_wait_segments: held until the flag reaches its target
    (a lower value does not release it), then exactly the listed byte ranges
    of the pinned buffer reach the device buffer (zero-length and adjacent
    segments included); every other byte keeps its old value, and the flag
    is left as the host wrote it."""
    lib = _native.load()
    print("case: host gate segments", flush=True)
    p = C.c_void_p()
    _native.check(lib.nsg_host_gate_alloc(C.byref(p)), "nsg_host_gate_alloc")
    flag = C.c_int32.from_address(p.value)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    n = 200_000
    src = torch.randint(0, 256, (n,), dtype=torch.uint8).pin_memory()
    dst = torch.full((n,), 7, dtype=torch.uint8, device="cuda")
    segs = [(0, 4096), (4096, 0), (4096, 160), (65536, 70_000), (199_984, 16)]
    offs = (C.c_int64 * len(segs))(*[o for o, _ in segs])
    lens = (C.c_int64 * len(segs))(*[l for _, l in segs])
    stream = torch.cuda.current_stream().cuda_stream
    try:
        flag.value = 4
        _native.check(lib.nsg_host_gate_wait_segments(p.value, 5, err.data_ptr(), 5_000_000,
                                                      src.data_ptr(), dst.data_ptr(), n, offs,
                                                      lens, len(segs), stream),
                      "nsg_host_gate_wait_segments")
        time.sleep(0.05)
        assert not torch.cuda.current_stream().query()      # 4 < 5: still held
        flag.value = 5
        torch.cuda.synchronize()
        assert int(err.item()) == 0 and flag.value == 5
        expect = torch.full((n,), 7, dtype=torch.uint8)
        for o, l in segs:
            expect[o:o + l] = src[o:o + l]
        assert torch.equal(dst.cpu(), expect)
    finally:
        torch.cuda.synchronize()
        _native.check(lib.nsg_host_gate_free(p.value), "nsg_host_gate_free")


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_pipelined_generate_equals_unpipelined(temperature):
    from nanosglang_amd.engine.spec_engine import SpecEngine
    print(f"case: pipelined generate T={temperature}", flush=True)
    gpu = _model()
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, 1000, n).tolist() for n in (20, 33, 5, 64, 12, 41)]
    max_new = [40, 17, 30, 9, 26, 33]
    outs, engines = [], []
    for pipeline in (True, False):
        eng = SpecEngine(gpu, draft_layers=2, num_speculative=4, num_blocks=128,
                         temperature=temperature, seed=9, max_batch=8, pipeline=pipeline)
        outs.append(eng.generate(prompts, max_new))
        engines.append(eng)
        print(f"  pipeline={pipeline}: steps {eng.stats['steps']} acceptance "
              f"{eng.stats['acceptance_rate']:.2f}", flush=True)
        assert eng.bm.num_free_blocks == 128 - 1     # the graphs' dummy padding page
        eng.check_device_flags()
    assert [len(o) for o in outs[0]] == max_new
    assert outs[0] == outs[1]
    assert engines[0].stats["steps"] == engines[1].stats["steps"]
    # a second pipelined run repeats itself (greedy) / continues its streams
    again = engines[0].generate(prompts, max_new)
    if temperature == 0.0:
        assert again == outs[0]


def test_pipelined_generate_releases_held_step_on_error():
    from nanosglang_amd.engine.spec_engine import SpecEngine
    print("case: pipelined generate, exception while a step is held", flush=True)
    gpu = _model()
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 1000, n).tolist() for n in (30, 18)]
    eng = SpecEngine(gpu, draft_layers=2, num_speculative=4, num_blocks=128, max_batch=2)
    ref = eng.generate(prompts, [30, 30])
    calls = {"n": 0}
    orig = eng._run_fill_next

    def failing(fill_next):
        calls["n"] += 1
        if calls["n"] == 2:            # the fill of a step that is queued behind the gate
            raise RuntimeError("injected")
        return orig(fill_next)

    eng._run_fill_next = failing
    t0 = time.perf_counter()
    with pytest.raises(RuntimeError, match="injected"):
        eng.generate(prompts, [30, 30])
    assert time.perf_counter() - t0 < 1.0             # released, not timed out
    eng._run_fill_next = orig
    assert calls["n"] == 2
    torch.cuda.synchronize()
    assert int(eng._gate_err.item()) == 0
    eng2 = SpecEngine(gpu, draft_layers=2, num_speculative=4, num_blocks=128, max_batch=2)
    assert eng2.generate(prompts, [30, 30]) == ref
