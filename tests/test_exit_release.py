"""CPU test of the release of library handles at interpreter exit
(engine_amd/kquant.py _release_all).

A child interpreter registers stand-in owners through the package's own
registry (no device, no library calls) and exits. Expected:
  - an owner kept alive only by a reference cycle (a test frame held by its
    exception's traceback, as `pytest.raises(...) as e` builds one) is still
    alive after its function returned, and is closed at exit;
  - every owner is closed once, dispatchers first and contexts last;
  - after the release, finalizers no longer reach the library.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

SCRIPT = r"""
import gc, weakref
from engine_amd import kquant as K

class Owner:
    def __init__(self, name, rank):
        self.name, self.handle = name, True
        K._own(self, rank)
    def close(self):
        if self.handle and K._live():
            print("close", self.name, flush=True)
            self.handle = False
    def __del__(self):
        self.close()

def failing_call():
    raise ValueError("expected")

def test_like():
    owner = Owner("cycle_decoder", K.RANK_DECODER)
    try:
        failing_call()
    except ValueError as exc:
        e = exc
    # e -> traceback -> this frame -> e: the owner lives until a collection
    return weakref.ref(owner)

gc.disable()
ref = test_like()
print("alive_after_return", ref() is not None, flush=True)
KEEP = [Owner("context", K.RANK_CONTEXT), Owner("weight", K.RANK_RESOURCE),
        Owner("dispatcher", K.RANK_DISPATCHER), Owner("cache", K.RANK_CACHE)]
import atexit
atexit.register(lambda: print("live_before_release", K._live(), flush=True))
"""


def test_owners_released_in_rank_order_at_exit():
    out = subprocess.run([sys.executable, "-c", SCRIPT], cwd=ROOT, capture_output=True, text=True, timeout=120,
                         env=dict(os.environ, HIP_VISIBLE_DEVICES=""))
    assert out.returncode == 0, out.stderr[-2000:]
    lines = out.stdout.split("\n")
    lines = [l for l in lines if l]
    assert lines[0] == "alive_after_return True"
    # the later-registered atexit handler runs first; the library release follows
    assert lines[1] == "live_before_release True"
    closes = [l.split()[1] for l in lines[2:]]
    assert closes[0] == "cycle_decoder"  # finalized by the collection
    assert closes[1:] == ["dispatcher", "cache", "weight", "context"]
