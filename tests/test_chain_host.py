"""The decode chain's host logic without a GPU: the checked step raises when the persistent
plan's error word is set (a hand-off wait that gave up), and queues without waiting inside a
graph capture."""
import pytest

from opentpu_amd import _lib
from opentpu_amd import chain as CH


class _Cuda:
    capturing = False
    synced = 0

    @classmethod
    def synchronize(cls):
        cls.synced += 1

    @classmethod
    def is_current_stream_capturing(cls):
        return cls.capturing


class _Torch:
    cuda = _Cuda


@pytest.fixture
def chain(monkeypatch):
    monkeypatch.setattr(_lib, "torch", lambda: _Torch)
    ch = CH.DecodeChain.__new__(CH.DecodeChain)
    ch._plan = (None, 4096)                   # a plan was built (its address is not read here)
    ch.x = None
    monkeypatch.setattr(CH.DecodeChain, "_queue", lambda self: None)
    ch.y = "y"
    return ch


def test_check_raises_on_the_error_word(chain, monkeypatch):
    monkeypatch.setattr(CH.DecodeChain, "chain_error", lambda self: 1)
    with pytest.raises(_lib.OtpuError, match="timed out") as e:
        chain.check()
    assert e.value.code == _lib.OTPU_ETIMEOUT
    with pytest.raises(_lib.OtpuError, match="timed out"):
        chain.step()
    assert chain.step(check=False) == "y"                 # unchecked: queued, no error read


def test_check_passes_on_a_clean_word(chain, monkeypatch):
    monkeypatch.setattr(CH.DecodeChain, "chain_error", lambda self: 0)
    n = _Cuda.synced
    assert chain.step() == "y"
    assert _Cuda.synced == n + 1                          # the check waited for the step


def test_no_check_inside_a_capture(chain, monkeypatch):
    monkeypatch.setattr(CH.DecodeChain, "chain_error", lambda self: 1)
    monkeypatch.setattr(_Cuda, "capturing", True)
    assert chain.step() == "y"                            # no sync may be issued while capturing


def _fits(hidden, q_dim, kv_dim, F, fmt="int4"):
    ch = CH.DecodeChain.__new__(CH.DecodeChain)
    ch.shape = CH.Shape(hidden=hidden, q_dim=q_dim, kv_dim=kv_dim, F=F)
    ch.fused, ch.fold, ch.fmt = True, True, fmt
    return ch.persistent_fits()


def test_persistent_fits_the_plan_rules():
    """Which chains take the persistent step: the Qwen3 shapes; a shape whose q/k/v rows span
    more workgroups than o's (o then also waits for k and v) while that wait's 2 kv_dim entries
    fit in 2048 (the GPU test runs it); not when they do not, and not past the compiled teams."""
    assert _fits(1024, 2048, 1024, 3072)                  # Qwen3-0.6B
    assert _fits(2048, 2048, 1024, 6144)                  # Qwen3-1.7B
    assert _fits(256, 512, 512, 768)                      # q/k/v on 96 workgroups, o on 64
    assert not _fits(256, 512, 1536, 768)                 # the same, with 3072 k and v entries
    assert not _fits(4096, 4096, 1024, 12288)             # hidden past 2048
    assert not _fits(1024, 2048, 1024, 3072, "int8")      # 4-bit weights only
    assert not _fits(1024, 2048, 1024, 3000)              # F a multiple of 256
