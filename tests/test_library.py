"""The C-ABI library builds, loads and exports every entry point the header
declares (no GPU needed: nothing here launches a kernel)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols(header='slimkv_hip.h'):
    text = re.sub(r'/\*.*?\*/', '', (ROOT / 'include' / header).read_text(), flags=re.S)
    return sorted(set(re.findall(r'\b(slimkv_[a-z0-9_]+)\s*\(', text)))


def test_every_header_is_checked():
    assert sorted(p.name for p in (ROOT / 'include').glob('*.h')) == ['slimkv_hip.h', 'slimkv_probe.h']


def test_header_declares_entry_points():
    names = declared_symbols()
    assert 'slimkv_latent_decode' in names and 'slimkv_attention_forward' in names


def test_library_exports_every_declared_symbol():
    from slimkv_amd import _lib
    handle = _lib.lib()
    for name in declared_symbols():
        assert hasattr(handle, name), name
        assert name in _lib.SIGNATURES, f'{name} has no ctypes signature'


def test_probe_library_exports_its_symbols_and_the_serving_library_none():
    """The measurement probes live in libslimkv_probe.so only."""
    from slimkv_amd import _lib
    probes = declared_symbols('slimkv_probe.h')
    assert probes == sorted(_lib.PROBE_SIGNATURES)
    handle = _lib.probe_lib()
    for name in probes:
        assert hasattr(handle, name), name
        assert not hasattr(_lib.lib(), name), f'{name} is exported by the serving library'


def STRUCTS(_lib):
    return (_lib.AttentionArgs, _lib.LatentDecodeArgs, _lib.ReconstructArgs, _lib.ReconDecodeArgs,
            _lib.RopeDecodeArgs, _lib.PrefillRopeArgs, _lib.MergeArgs, _lib.PrefillAttentionArgs, _lib.DownProjectArgs,
            _lib.BeaconPagesArgs, _lib.RawPagesArgs, _lib.PagedLatentDecodeArgs, _lib.PageRows, _lib.LinearRowsArgs,
            _lib.DecodeQKVArgs, _lib.EagerAttentionArgs, _lib.PagedStepRowsArgs)


def test_struct_layouts_match_header_field_order():
    """ctypes mirrors list the header's fields in order with matching widths."""
    from slimkv_amd import _lib
    header = (ROOT / 'include' / 'slimkv_hip.h').read_text()
    for struct in STRUCTS(_lib):
        body = re.search(r'typedef struct %s \{(.*?)\}' % struct.__name__, header, re.S).group(1)
        body = re.sub(r'/\*.*?\*/', '', body, flags=re.S)
        fields = re.findall(r'\*?\s*([a-z_][a-z0-9_]*)\s*(?=[,;])', body)
        assert fields == [f[0] for f in struct._fields_], struct.__name__


def test_struct_offsets_match_the_c_compiler(tmp_path):
    """sizeof and every offsetof of each argument struct, as gcc lays out the
    header, equal the ctypes mirror's."""
    import shutil
    import subprocess
    from slimkv_amd import _lib
    if shutil.which('gcc') is None:
        pytest.skip('gcc not available')
    lines = []
    for struct in STRUCTS(_lib):
        name = struct.__name__
        lines.append(f'printf("%s size %zu\\n", "{name}", sizeof({name}));')
        for field, _ in struct._fields_:
            lines.append(f'printf("%s %s %zu\\n", "{name}", "{field}", offsetof({name}, {field}));')
    src = tmp_path / 'layout.c'
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "slimkv_hip.h"\nint main(void){\n' +
                   '\n'.join(lines) + '\nreturn 0;}\n')
    exe = tmp_path / 'layout'
    subprocess.run(['gcc', '-I', str(ROOT / 'include'), str(src), '-o', str(exe)], check=True)
    got = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split('\n')
    want = []
    for struct in STRUCTS(_lib):
        want.append(f'{struct.__name__} size {ctypes.sizeof(struct)}')
        want += [f'{struct.__name__} {f} {getattr(struct, f).offset}' for f, _ in struct._fields_]
    assert got[:-1] == want


def test_errors_are_reported_without_a_gpu():
    from slimkv_amd import _lib
    a = _lib.AttentionArgs()
    assert _lib.lib().slimkv_attention_workspace(ctypes.byref(a)) == 0
    assert b'null' in _lib.lib().slimkv_last_error()
    with pytest.raises(ValueError):
        _lib.check(-1)
