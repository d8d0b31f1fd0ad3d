"""The C ABI boundary without a GPU: the libraries load, export every symbol
the headers declare, and the host-only entry points behave as specified."""
import ctypes
import subprocess

import numpy as np
import pytest


def test_hsamp_exports_every_declared_symbol(pkg):
    hs = pkg.hsamp
    L = hs.lib()
    names = hs.declared_symbols()
    assert len(names) >= 9
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/ultima_hsamp.h but not exported"
    assert "ultima_hsamp_run_noalloc" not in names


def test_noalloc_library_exports_its_entry_and_holds_the_array(pkg):
    """The allocation-free entry is exported by its own library, whose device
    array (the only one) is not in the main library."""
    hs = pkg.hsamp
    L = hs.noalloc_lib()
    names = sorted(set(hs.declared_symbols(hs.NOALLOC_HEADER)) - set(hs.declared_symbols()))
    assert names == ["ultima_hsamp_run_noalloc"]
    for n in names:
        assert hasattr(L, n)
    main = hs.lib()
    assert not hasattr(main, "ultima_hsamp_run_noalloc")


def test_version_and_status_strings(pkg):
    L = pkg.hsamp.lib()
    assert L.ultima_hsamp_version() == 1
    for st in (0, -1, -2, -3, -4, -5, -6):
        assert L.ultima_hsamp_status_str(st).decode() not in ("", "unknown status")
    assert L.ultima_hsamp_status_str(-99).decode() == "unknown status"


def test_params_default_and_identity_match_reference(pkg, orc):
    hs = pkg.hsamp
    L = hs.lib()
    for fn, ref in ((L.ultima_hsamp_params_default, orc.default_params()),
                    (L.ultima_hsamp_params_identity, orc.identity_params())):
        p = hs.Params()
        fn(ctypes.byref(p))
        for k, v in ref.items():
            assert getattr(p, k) == pytest.approx(np.float32(v)) if isinstance(v, float) else getattr(p, k) == v, k
        assert p.hist_len == 0 and p.bias_count == 0


@pytest.mark.parametrize("seed", [0, 1, 42, 5489, 123456])
def test_uniform_from_u64_is_generate_canonical(pkg, orc, seed):
    L = pkg.hsamp.lib()
    x = orc.mt19937_64_nth(seed, 1)
    assert L.ultima_hsamp_uniform_from_u64(x) == orc.u_from_seed(seed)


def test_uniform_from_u64_clamps_below_one(pkg):
    L = pkg.hsamp.lib()
    assert L.ultima_hsamp_uniform_from_u64(2**64 - 1) == np.nextafter(1.0, 0.0)
    assert L.ultima_hsamp_uniform_from_u64(0) == 0.0


def test_create_rejects_bad_arguments(pkg):
    L = pkg.hsamp.lib()
    h = ctypes.c_void_p()
    assert L.ultima_hsamp_create(0, 0, 100, ctypes.byref(h)) == -1
    assert L.ultima_hsamp_create(0, 10, 0, ctypes.byref(h)) == -1
    assert L.ultima_hsamp_create(0, 10, 1 << 25, ctypes.byref(h)) == -5
    assert L.ultima_hsamp_create(0, 10, 100, None) == -1
    assert L.ultima_hsamp_destroy(None) == 0
    assert L.ultima_hsamp_run(None, None, None) == -1


def test_create_without_gfx950_reports_no_device(pkg):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = pkg.hsamp.lib()
    h = ctypes.c_void_p()
    assert L.ultima_hsamp_create(0, 10, 100, ctypes.byref(h)) == -6
    assert not h.value


def test_cpp_dropin_exports_reference_interface(pkg):
    so = pkg.hsamp.PKG / "libultima_sampler.so"
    out = subprocess.run(["nm", "-DC", "--defined-only", str(so)], capture_output=True, text=True,
                         check=True).stdout
    for sym in ("ultima::sampler::sample(std::span<float, 18446744073709551615ul>, "
                "ultima::sampler::SamplerParams const&, ultima::sampler::SamplerContext&)",
                "ultima::sampler::argmax(std::span<float const, 18446744073709551615ul>)",
                "ultima::sampler::SamplerParams::identity()",
                "ultima::sampler::SamplerContext::SamplerContext(unsigned long)",
                "ultima::sampler::SamplerContext::SamplerContext()",
                "ultima::sampler::SamplerContext::push_recent(int)",
                "ultima::sampler::SamplerContext::set_recent(std::span<int const, 18446744073709551615ul>)"):
        assert sym in out, sym


def test_product_does_not_link_the_oracle(pkg):
    for so in ("libultima_hsamp.so", "libultima_sampler.so"):
        out = subprocess.run(["ldd", str(pkg.hsamp.PKG / so)], capture_output=True, text=True).stdout
        assert "orc_sampler" not in out and "ref_sampler" not in out
        syms = subprocess.run(["nm", "-D", str(pkg.hsamp.PKG / so)], capture_output=True,
                              text=True).stdout
        assert "orc_" not in syms and "ref_sample" not in syms


def test_struct_layouts_match_the_header(pkg, tmp_path):
    """The binding's ctypes structs have the C header's size and field offsets
    (a C program built against include/ultima_hsamp.h prints them)."""
    hs = pkg.hsamp
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    structs = {"ultima_hsamp_params": hs.Params, "ultima_hsamp_batch": hs.Batch, "ultima_hsamp_head": hs.Head,
               "ultima_hsamp_verify": hs.Verify, "ultima_hsamp_commit": hs.Commit}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "ultima_hsamp.h"', 'int main(void) {']
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines += ['return 0;', '}']
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(root / "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for f, _ in py._fields_:
            assert got[(cname, f)] == getattr(py, f).offset, f"{cname}.{f}"


def test_history_push_rejects_bad_arguments(pkg):
    """Argument checks run before any device work (no GPU needed)."""
    hs = pkg.hsamp
    L = hs.lib()
    p = ctypes.c_void_p(16)   # never dereferenced: every call below fails its checks first
    assert L.ultima_hsamp_history_push(None, 8, p, p, 1, 4, None) == hs.ERR_INVALID
    assert L.ultima_hsamp_history_push(p, 8, None, p, 1, 4, None) == hs.ERR_INVALID
    assert L.ultima_hsamp_history_push(p, 8, p, None, 1, 4, None) == hs.ERR_INVALID
    assert L.ultima_hsamp_history_push(p, 8, p, p, 0, 4, None) == hs.ERR_INVALID        # no rows
    assert L.ultima_hsamp_history_push(p, 8, p, p, 1, 5, None) == hs.ERR_INVALID        # keep > stride / 2
    assert L.ultima_hsamp_history_push(p, 8, p, p, 1, 0, None) == hs.ERR_INVALID        # keep < 1
    assert L.ultima_hsamp_history_push(p, 1, p, p, 1, 1, None) == hs.ERR_INVALID        # stride < 2


def test_decode_commit_rejects_bad_arguments(pkg):
    """Argument checks run before any device work (no GPU needed)."""
    hs = pkg.hsamp
    L = hs.lib()
    p = ctypes.c_void_p(16)   # never dereferenced: every call below fails its checks first
    stop = (ctypes.c_int32 * 9)(*range(9))
    assert L.ultima_hsamp_decode_commit(None, 8, p, p, p, None, 1, 4, None, 0, None) == hs.ERR_INVALID
    assert L.ultima_hsamp_decode_commit(p, 8, None, p, p, None, 1, 4, None, 0, None) == hs.ERR_INVALID
    assert L.ultima_hsamp_decode_commit(p, 8, p, None, p, None, 1, 4, None, 0, None) == hs.ERR_INVALID
    assert L.ultima_hsamp_decode_commit(p, 8, p, p, None, None, 1, 4, None, 0, None) == hs.ERR_INVALID  # active
    assert L.ultima_hsamp_decode_commit(p, 8, p, p, p, None, 0, 4, None, 0, None) == hs.ERR_INVALID     # no rows
    assert L.ultima_hsamp_decode_commit(p, 8, p, p, p, None, 1, 5, None, 0, None) == hs.ERR_INVALID     # keep
    assert L.ultima_hsamp_decode_commit(p, 8, p, p, p, None, 1, 4, None, 2, None) == hs.ERR_INVALID     # no ids
    assert L.ultima_hsamp_decode_commit(p, 8, p, p, p, None, 1, 4, stop, 9, None) == hs.ERR_INVALID     # > 8 ids
    assert L.ultima_hsamp_decode_commit(p, 8, p, p, p, None, 1, 4, stop, -1, None) == hs.ERR_INVALID


def test_run_commit_rejects_bad_arguments(pkg):
    """The commit's checks (decode_commit's) run before the batch is looked at
    (no GPU needed); a write-back batch is refused."""
    hs = pkg.hsamp
    L = hs.lib()
    h = ctypes.c_void_p(16)   # never dereferenced: every call below fails its checks first
    p = 16
    stop = (ctypes.c_int32 * 9)(*range(9))

    def mk(**kw):
        c = hs.Commit()
        c.hist, c.hist_stride, c.hist_len_dev, c.active, c.keep = p, 8, p, p, 4
        for k, x in kw.items():
            setattr(c, k, x)
        return c

    b = hs.Batch()
    assert L.ultima_hsamp_run_commit(h, ctypes.byref(b), None, None) == hs.ERR_INVALID
    for bad in (dict(hist=None), dict(hist_len_dev=None), dict(active=None), dict(hist_stride=1), dict(keep=0),
                dict(keep=5), dict(n_stop=2), dict(n_stop=9, stop_ids=ctypes.cast(stop, ctypes.c_void_p)),
                dict(n_stop=-1)):
        assert L.ultima_hsamp_run_commit(h, ctypes.byref(b), ctypes.byref(mk(**bad)), None) == hs.ERR_INVALID, bad
    b.flags = hs.WRITEBACK
    assert L.ultima_hsamp_run_commit(h, ctypes.byref(b), ctypes.byref(mk()), None) == hs.ERR_UNSUPPORTED
    assert L.ultima_hsamp_run_commit(None, None, ctypes.byref(mk()), None) == hs.ERR_INVALID


def test_verify_block_rejects_bad_arguments(pkg):
    """Argument checks run before any device work (no GPU needed); the
    workspace size is n_pos rows of hist_len + n_pos - 1 ids plus n_pos."""
    hs = pkg.hsamp
    L = hs.lib()
    assert L.ultima_hsamp_verify_work_ints(5, 100) == 5 * 104 + 5
    assert L.ultima_hsamp_verify_work_ints(1, 0) == 1 + 1
    assert L.ultima_hsamp_verify_work_ints(0, 10) == -1
    assert L.ultima_hsamp_verify_work_ints(3, -1) == -1
    h = ctypes.c_void_p(16)   # never dereferenced
    p = 16
    par = (hs.Params * 1)()

    def mk(**kw):
        v = hs.Verify()
        v.n_pos, v.vocab, v.dtype, v.logits, v.logits_stride = 4, 100, hs.F32, p, 100
        v.draft, v.hist, v.hist_len, v.u, v.params = p, p, 10, p, par
        v.work, v.out_tokens, v.out_count = p, p, p
        for k, x in kw.items():
            setattr(v, k, x)
        return v

    assert L.ultima_hsamp_verify_block(None, ctypes.byref(mk()), None) == hs.ERR_INVALID
    assert L.ultima_hsamp_verify_block(h, None, None) == hs.ERR_INVALID
    for bad in (dict(n_pos=0), dict(hist_len=-1), dict(vocab=0), dict(logits=None), dict(u=None), dict(work=None),
                dict(out_tokens=None), dict(out_count=None), dict(draft=None), dict(hist=None),
                dict(params=ctypes.POINTER(hs.Params)())):
        assert L.ultima_hsamp_verify_block(h, ctypes.byref(mk(**bad)), None) == hs.ERR_INVALID, bad
