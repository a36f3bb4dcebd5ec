"""The output head at a real vocabulary on the GPU: 248,320 rows (the reference's
Qwen3.5 vocabulary, tests/tiny_moe.py:121; src/engine.mm:1634-1638), hidden 4096 with an
affine head (bf16 scales and biases, as tools/convert.py stores them) and hidden 5120 with
a native int15 head and an MTP head (src/engine.mm:398,534).

- rl_head at 1, 5 and 16 rows: logits on sampled columns (the first and last four and 248
  drawn ones) within 1e-3 of the fp64 product of the normed rows.
- rl_top_k_device and rl_argmax against rl_top_k on the host copy: exact ids and values,
  over one row and over all 16 rows of the logits (n = 16 x 248,320 at k = 256: several
  merge passes).
- rl_argmax after rl_head on a side stream (the top-k must run after the head's kernels).
- rl_draft_head with a draft vocabulary and, for the native head, a tail
  (src/engine.mm:1425-1458): the main and tail rows of the head; the row normed with
  mtp.norm in the file with an MTP head, with final_norm otherwise.
"""

import numpy as np
import pytest

import oracle as O
import oracle.engine as OE
from raceline_amd import lib
from raceline_amd.model import Engine, copy_from_device_ptr, top_k
from tests import model_files as MF
from tests.qdata import to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-3
VOCAB = 248320


def _sync():
    import torch

    torch.cuda.synchronize()


@pytest.fixture(scope="module", params=[(4096, None), (5120, "int15")], ids=["h4096_q4a_bf16", "h5120_int15_mtp"])
def head_model(request, tmp_path_factory):
    hidden, book = request.param
    path = str(tmp_path_factory.mktemp("head") / f"head_{hidden}.rlm")
    print(f"[head] writing a {VOCAB} x {hidden} head ({book or 'q4a bf16'})", flush=True)
    return MF.write_head_model(path, hidden, VOCAB, native_book=book, seed=hidden, mtp=book is not None)


def _sample_cols(rng, n):
    return np.unique(np.concatenate([np.arange(4), np.arange(n - 4, n), rng.integers(0, n, 248)]))


def _head_ref(m, xn, cols):
    if "lm_head" in m.affine:
        q, sb, bb, _ = m.affine["lm_head"]
        return O.linear_affine_f64(xn, q[cols], sb[cols], bb[cols], "bf16")
    codes, s, _, _ = m.native["lm_head"]
    return O.linear_native_f64(xn, codes[cols], s[cols], m.book)


def _norm_weight(m, name):
    w = m.floats[name]
    if "lm_head" in m.native:
        w = (w * m.native["lm_head"][2]).astype(np.float32)   # folded with the head's column scales
    return w


def test_head_logits_and_top_k(gpu, head_model):
    m = head_model
    H = m.cfg["hidden_size"]
    rng = np.random.default_rng(H)
    with Engine(m.path, max_chunk=16) as e:
        assert e.vocab == VOCAB and e.logits_stride == VOCAB
        for rows in (1, 5, 16):
            h0 = rng.standard_normal((rows, H)).astype(np.float32)
            print(f"[head] H={H} rows={rows}", flush=True)
            logits = e.head(to_dev(h0, gpu))
            _sync()
            got = logits.cpu().numpy()
            xn = OE.rms_norm_f16(h0, _norm_weight(m, "final_norm"), m.cfg["rms_norm_eps"])
            cols = _sample_cols(rng, VOCAB)
            O.check_close(got[:, cols], _head_ref(m, xn, cols), TOL, f"head H={H} rows={rows}")
            assert np.isfinite(got).all()
            for k in (1, 50, 256):
                ids, vals = e.top_k_device(logits[0].contiguous(), k)
                rid, rvals = top_k(got[0], k)
                assert ids == list(rid), f"top-{k} of row 0, rows={rows}"
                np.testing.assert_array_equal(np.float32(vals), rvals)
            assert e.argmax() == int(np.argmax(got[0]))
        # all 16 rows at once: 16 x 248,320 candidates, the largest n the engine takes
        ids, vals = e.top_k_device(logits.reshape(-1).contiguous(), 256)
        rid, rvals = top_k(got.reshape(-1), 256)
        assert ids == list(rid)
        np.testing.assert_array_equal(np.float32(vals), rvals)


def test_argmax_follows_the_heads_stream(gpu, head_model):
    """rl_argmax runs on the stream of the last rl_head: called at once after a head on a
    side stream, it still sees that head's logits, not the ones before."""
    import torch

    m = head_model
    H = m.cfg["hidden_size"]
    rng = np.random.default_rng(H + 1)
    with Engine(m.path, max_chunk=16) as e:
        ha = to_dev(rng.standard_normal((1, H)).astype(np.float32), gpu)
        hb = to_dev(rng.standard_normal((1, H)).astype(np.float32), gpu)
        first = e.head(ha).cpu().numpy()[0]
        _sync()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            # rl_head itself (Engine.head waits for its stream to copy the logits out)
            ptr = lib.load().rl_head(e._e, hb.data_ptr(), hb.stride(0), 1, side.cuda_stream)
            assert ptr
            got = e.argmax()              # at once, with the head's kernels still queued
        _sync()
        want = int(np.argmax(copy_from_device_ptr(ptr, (1, VOCAB)).cpu().numpy()[0]))
        assert want != int(np.argmax(first)), "the two rows should have different argmax"
        assert got == want


def test_draft_head_main_and_tail(gpu, head_model):
    import torch

    m = head_model
    H = m.cfg["hidden_size"]
    native = "lm_head" in m.native
    rng = np.random.default_rng(H + 2)
    h_row = rng.standard_normal(H).astype(np.float32)
    with Engine(m.path, max_chunk=16) as e:
        e.set_draft_vocab(150000)
        e.set_draft_tail(248000)
        main, tail = e.draft_main, e.draft_tail
        assert main == 150016
        assert tail == (247808 if native else -1)           # a tail only for native heads
        d = e.draft_head(to_dev(h_row, gpu))
        _sync()
        assert d.numel() == e.draft_vocab == main + (VOCAB - tail if native else 0)
        if "mtp.norm" in m.floats:
            # the MTP head's row: normed with mtp.norm folded with the head's column scales
            xn = OE.rms_norm_f16(h_row[None, :], _norm_weight(m, "mtp.norm"), m.cfg["rms_norm_eps"])
            idx = _sample_cols(rng, d.numel())
            rows = np.where(idx < main, idx, idx - main + tail)
            O.check_close(d.cpu().numpy()[idx][None, :], _head_ref(m, xn, rows), TOL, f"draft head H={H}")
        else:
            full = e.head(to_dev(h_row[None, :].copy(), gpu))[0]
            _sync()
            assert torch.equal(d, full[:main])
