"""Restore-pipeline bookkeeping on the CPU: a replaced pipeline stays alive
while leased or busy; event-timed metric rows are written once their events
complete (worker.py:574-617)."""
import json
import threading

import pytest

from origami_amd.restore_pipeline import PipelineRegistry


class FakePipe:
    def __init__(self, index, slot_bytes):
        self.index = index
        self.slot_bytes = slot_bytes
        self.busy = False

    def idle(self):
        return not self.busy


def _registry():
    made = []

    def factory(index, slot_bytes):
        made.append(FakePipe(index, slot_bytes))
        return made[-1]
    return PipelineRegistry(factory), made


def test_same_or_smaller_request_reuses_pipeline():
    reg, made = _registry()
    with reg.lease(0, 100) as a:
        pass
    with reg.lease(0, 100) as b:
        pass
    with reg.lease(0, 50) as c:
        pass
    assert a is b is c and len(made) == 1
    assert reg.retired() == []


def test_larger_request_retires_old_pipeline_while_leased():
    reg, made = _registry()
    old = reg.acquire(0, 100)          # a thread is still using it
    with reg.lease(0, 200) as new:     # another request needs bigger slots
        assert new is not old and new.slot_bytes == 200
        assert reg.current()[0] is new
        assert old in reg.retired()    # not dropped: still leased
    reg.prune()
    assert old in reg.retired()
    reg.release(old)                   # last lease gone and idle -> released
    assert old not in reg.retired()


def test_retired_pipeline_kept_until_its_work_completes():
    reg, _ = _registry()
    with reg.lease(0, 100) as old:
        old.busy = True                # queued GPU work still pending
    with reg.lease(0, 300):
        pass
    assert old in reg.retired()
    reg.prune()
    assert old in reg.retired()
    old.busy = False
    reg.prune()
    assert reg.retired() == []


def test_devices_are_independent():
    reg, made = _registry()
    with reg.lease(0, 100) as a, reg.lease(1, 400) as b:
        assert a is not b
    with reg.lease(0, 100) as a2:
        assert a2 is a
    assert set(reg.current()) == {0, 1}


def test_release_without_lease_raises():
    reg, _ = _registry()
    pipe = reg.acquire(0, 10)
    reg.release(pipe)
    with pytest.raises(RuntimeError):
        reg.release(pipe)


def test_concurrent_growing_leases_never_drop_a_leased_pipeline():
    reg, made = _registry()
    errors = []
    held = []
    lock = threading.Lock()

    def worker(k):
        try:
            for i in range(200):
                with reg.lease(0, 1 + (k * 200 + i) % 97) as pipe:
                    with lock:
                        held.append(pipe)
                    # while leased, the pipeline is current or retired
                    if pipe is not reg.current().get(0) and pipe not in reg.retired():
                        errors.append("leased pipeline dropped")
                    with lock:
                        held.remove(pipe)
        except Exception as exc:  # noqa: BLE001
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors
    reg.prune()
    assert reg.retired() == []  # nothing leased or busy is left behind


class FakeEvent:
    def __init__(self, t, done=True):
        self.t = t
        self.done = done
        self.synced = False

    def query(self):
        return self.done

    def synchronize(self):
        self.synced = True
        self.done = True

    def elapsed_time(self, other):
        return other.t - self.t


def test_deferred_metric_rows(tmp_path):
    from origami_amd.config import OrigamiConfig
    from origami_amd.metadata import LayerPayload, OrigamiRestoreRequest
    from origami_amd.store import InMemoryOrigamiStore
    from origami_amd.worker import OrigamiConnectorWorker

    cfg = OrigamiConfig(quantizer="raw_byte_planes", metrics_dir=str(tmp_path),
                        lossless_cpu_backend="zlib", allow_zlib_fallback=True,
                        bitunpack_device="auto")
    w = OrigamiConnectorWorker(cfg, InMemoryOrigamiStore())
    restore = OrigamiRestoreRequest(request_id="r1", cache_key="k", block_ids_per_group=((0,),),
                                    num_tokens=16)
    lp = LayerPayload(layer_name="model.layers.0.self_attn", quantizer="raw_byte_planes",
                      quant_metadata={}, chunks=[])
    done_row = ("bitunpack_cuda", restore, lp,
                {"bytes": 2_000_000, "input_bytes": 1_000_000,
                 "_cuda_start_event": FakeEvent(1.0), "_cuda_end_event": FakeEvent(3.0)})
    late_end = FakeEvent(5.0, done=False)
    late_row = ("h2d_copy", restore, lp,
                {"bytes_copied": 4_000_000, "_cuda_start_event": FakeEvent(1.0),
                 "_cuda_end_event": late_end})
    w._flush_pending_cuda_metrics([done_row, late_row])
    rows = [json.loads(x) for x in (tmp_path / "origami_metrics.jsonl").read_text().splitlines()]
    assert [r["type"] for r in rows] == ["bitunpack_cuda"]
    r = rows[0]
    assert r["ms"] == 2.0 and r["request_id"] == "r1" and r["layer_name"] == lp.layer_name
    assert r["gbps"] == pytest.approx(2_000_000 * 8 / 2.0 / 1e6)
    assert r["input_gbps"] == pytest.approx(1_000_000 * 8 / 2.0 / 1e6)
    assert not any(k.startswith("_cuda") for k in r)
    # the unfinished row is written by a later flush once its event completes
    w._flush_pending_cuda_metrics(None)
    assert len((tmp_path / "origami_metrics.jsonl").read_text().splitlines()) == 1
    late_end.done = True
    w._flush_pending_cuda_metrics(None)
    rows = [json.loads(x) for x in (tmp_path / "origami_metrics.jsonl").read_text().splitlines()]
    assert rows[1]["type"] == "h2d_copy" and rows[1]["h2d_ms"] == 4.0
    assert rows[1]["h2d_gbps"] == pytest.approx(4_000_000 * 8 / 4.0 / 1e6)
    assert rows[1]["timing_complete"] is True
    # final flush waits on events still pending
    pending = FakeEvent(2.5, done=False)
    w._flush_pending_cuda_metrics([("restore_materialize", restore, lp,
                                    {"_cuda_start_event": FakeEvent(0.5),
                                     "_cuda_end_event": pending})], final=True)
    assert pending.synced
    w._executor.shutdown()
