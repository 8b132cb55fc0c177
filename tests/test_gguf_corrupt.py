"""The host GGUF reader on damaged files: every violation gguf_open rejects
(gguf.c:272-278 header and counts, gguf.c:343-351 tensor data inside the file)
comes back as an error with the reference's message, and an image cut short
at any point of its header, metadata, descriptors or data is refused rather
than read past its end."""
import ctypes as C
import struct

import numpy as np
import pytest

import fwgpu


def small_image() -> bytes:
    sp = fwgpu.spec(64, 128, 1, 2, 2, 50, 16, 10000.0, seed=3)
    H = fwgpu.host_lib()
    n = H.fwh_synth_size(C.byref(sp))
    buf = C.create_string_buffer(n)
    assert H.fwh_synth_write(C.byref(sp), buf, n) == n
    return buf.raw


def open_err(image: bytes) -> str:
    with pytest.raises(ValueError) as e:
        fwgpu.HostModel(image=image).close()
    return str(e.value)


def tensor_offset_field(image: bytes, name: bytes) -> int:
    """Byte position of a tensor descriptor's data offset: name, n_dims (u32),
    dims (u64 each), ggml type (u32), then the u64 offset (gguf.c:296-312)."""
    p = image.index(struct.pack("<Q", len(name)) + name) + 8 + len(name)
    n_dims = struct.unpack_from("<I", image, p)[0]
    return p + 4 + 8 * n_dims + 4


def test_valid_image_opens():
    with fwgpu.HostModel(image=small_image()) as host:
        assert host.cfg.n_embd == 64 and host.n_tensors > 0


def test_bad_magic_and_header():
    img = small_image()
    assert "not a valid GGUF header" in open_err(b"GGUG" + img[4:])
    for version in (1, 4):
        assert "unsupported GGUF version" in open_err(img[:4] + struct.pack("<I", version) + img[8:])
    assert "unsupported GGUF version/counts" in open_err(img[:8] + struct.pack("<Q", 10_000_001) + img[16:])
    assert "unsupported GGUF version/counts" in open_err(img[:16] + struct.pack("<Q", 10_000_001) + img[24:])


def test_tensor_offset_and_size_past_end_of_file():
    img = bytearray(small_image())
    with fwgpu.HostModel(image=bytes(img)) as host:
        data_size = host.data_size
    f = tensor_offset_field(bytes(img), b"output.weight")
    bad = bytearray(img)
    struct.pack_into("<Q", bad, f, data_size + 64)
    assert "offset outside file" in open_err(bytes(bad))
    bad = bytearray(img)
    struct.pack_into("<Q", bad, f, data_size - 32)           # starts inside, ends past the end
    assert "extends beyond file" in open_err(bytes(bad))


def test_every_truncation_is_refused():
    img = small_image()
    with fwgpu.HostModel(image=img) as host:
        data_start = len(img) - host.data_size
        data_end = data_start + max(host.tensors[i].offset + host.tensors[i].byte_size
                                    for i in range(host.n_tensors))
    # past data_end only the alignment padding of the last tensor is cut: still valid
    cuts = sorted(set(list(range(0, 64)) + list(range(64, data_start, 13)) +
                      [data_start - 1, data_start, data_start + 1, data_end - 1]))
    for cut in cuts:
        open_err(img[:cut])
    with fwgpu.HostModel(image=img[:data_end]):
        pass
    # random byte damage in the descriptors either opens or is refused, never crashes
    rng = np.random.default_rng(4)
    for _ in range(200):
        bad = bytearray(img[:data_start])
        for i in rng.integers(24, data_start, 4):
            bad[i] = int(rng.integers(0, 256))
        try:
            fwgpu.HostModel(image=bytes(bad) + img[data_start:]).close()
        except ValueError:
            pass
