"""Out-of-memory classification on the GPU (native_backend.rs:294-300,
gpu-runtime lib.rs:199-223) and the actionable message of a trainer that does
not fit (training.rs:100-146): an impossible allocation and an impossible
trainer raise OutOfMemory, free what they took, and leave the device usable
for a normal trainer in the same process."""
import ctypes as C

import numpy as np
import pytest

from tatara_amd import _lib
from tatara_amd.synthetic import small_spec, structured_batch
from tatara_amd.trainer import LayerStackConfig, LayerStackTrainer, Sigmoid, oom_remedy

@pytest.mark.gpu
def test_malloc_beyond_hbm_is_out_of_memory(gpu):
    lib = _lib.load()
    p = C.c_void_p()
    st = lib.tatara_malloc(C.byref(p), 1 << 50)  # 1 PiB
    assert st == -2, (st, lib.tatara_last_error())
    assert p.value is None
    assert "out of memory" in lib.tatara_last_error().decode().lower()
    with pytest.raises(_lib.OutOfMemory):
        _lib.check(st)
    # the runtime keeps working: a small allocation round-trips
    _lib.check(lib.tatara_malloc(C.byref(p), 1 << 20))
    host = np.arange(1 << 18, dtype=np.int32)
    back = np.zeros_like(host)
    _lib.check(lib.tatara_memcpy_htod(p, host.ctypes.data, host.nbytes))
    _lib.check(lib.tatara_memcpy_dtoh(back.ctypes.data, p, host.nbytes))
    _lib.check(lib.tatara_free(p))
    assert np.array_equal(host, back)


@pytest.mark.gpu
def test_trainer_too_large_is_out_of_memory_and_device_stays_usable(gpu):
    # LS1536 shapes with a batch whose raw-sum buffers alone (2^26 x 1536 f32
    # x 2) exceed the 288 GB of HBM: create allocates the parameter groups
    # and the smaller workspaces, then fails, and frees them all
    big = LayerStackConfig(ft_in=73305, max_active=40, piece_inputs=1629, ft_out=1536, l1_out=16, l2_out=32,
                           num_buckets=8, max_batch=1 << 26, optimizer="ranger")
    with pytest.raises(_lib.OutOfMemory) as ei:
        LayerStackTrainer(big)
    msg = str(ei.value)
    assert "hipMalloc" in msg
    assert msg.endswith(oom_remedy(big).splitlines()[-1])
    assert "batch-size=67108864, --ft-out=1536" in msg and "--fp16-opt-state" in msg

    # a normal trainer creates and trains on the same device afterwards, and
    # gives the same result as a second one (nothing left over from the failure)
    spec = small_spec(king_buckets=10, piece_inputs=64, max_active=40)
    cfg = LayerStackConfig(ft_in=spec["ft_in"], max_active=40, piece_inputs=64, ft_out=256, l1_out=16, l2_out=32,
                           num_buckets=8, max_batch=256, optimizer="ranger")
    batch, bucket = structured_batch(256, spec, num_buckets=8, seed=5, nnz_min=30)
    out = []
    for _ in range(2):
        with LayerStackTrainer(cfg) as t:
            for _ in range(3):
                t.train_step(batch, bucket, 1e-3, 0.0, Sigmoid(1.0 / 290.0))
            loss = t.flush_pending_loss()
            out.append((loss, t.get("ft_w"), t.get("l1_w")))
    assert np.isfinite(out[0][0]) and out[0][0] > 0
    assert out[0][0] == out[1][0]
    assert np.array_equal(out[0][1], out[1][1]) and np.array_equal(out[0][2], out[1][2])


def test_oom_remedy_text():
    cfg = LayerStackConfig(ft_in=73305, max_active=40, piece_inputs=1629, ft_out=1536, l1_out=16, l2_out=32,
                           num_buckets=8, max_batch=65536, optimizer="ranger").all_optim()
    text = oom_remedy(cfg)
    assert text.splitlines()[0] == ("GPU out of memory while allocating training buffers (batch-size=65536, "
                                    "--ft-out=1536, ft-fp16=true, ft-fp16-out=true, fp16-opt-state=true).")
    # f16 moments already on: not offered again
    assert "--fp16-opt-state" not in text.split("\n", 1)[1]
    assert text.splitlines()[-1] == "  - smaller `--batch-size`"
