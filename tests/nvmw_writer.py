"""Writes .nvmw files for the tests, in the layout jinf's prepare_model tool
produces (tools/prepare_model.cpp:106-300, bundle section :296-490; record
layouts include/jinf/nvmw.h:24-100): a 4096-byte header, at 4096 the layer
descriptors then the 200-byte tensor entries, the hot region at the next 4 KiB
boundary with every tensor padded to 4 KiB, then each layer's cold region
starting on a 4 KiB boundary, and, for version 2, 4 KiB-padded neuron bundles
followed by the bundle index.  All little-endian."""
import struct

MAGIC = 0x574D564E
HEADER_BYTES, LAYER_BYTES, ENTRY_BYTES = 4096, 24, 200


def align4k(n):
    return (n + 4095) & ~4095


def header_bytes(h):
    b = bytearray(HEADER_BYTES)
    struct.pack_into("<IIII", b, 0, h["magic"], h["version"], h["n_layers"], h["n_tensors"])
    struct.pack_into("<6Q", b, 16, h["index_offset"], h["index_size"], h["hot_offset"],
                     h["hot_size"], h["cold_start_offset"], h["cold_total_size"])
    struct.pack_into("<6I", b, 64, h["n_embd"], h["n_heads"], h["n_heads_kv"], h["n_ff"],
                     h["n_vocab"], h["n_ctx_train"])
    struct.pack_into("<ffiI", b, 88, h["rope_freq_base"], h["rms_norm_eps"], h["primary_type"], 0)
    struct.pack_into("<Q", b, 104, h["bundle_index_offset"])
    return bytes(b)


def entry_bytes(name, qtype, shape, n_dims, offset, n_bytes, layer_index, is_hot):
    b = bytearray(ENTRY_BYTES)
    nb = name.encode()[:127]
    b[:len(nb)] = nb
    struct.pack_into("<i", b, 128, qtype)
    struct.pack_into("<4q", b, 136, *(list(shape) + [0] * (4 - len(shape))))
    struct.pack_into("<I", b, 168, n_dims)
    struct.pack_into("<QQiB", b, 176, offset, n_bytes, layer_index, is_hot)
    return bytes(b)


def write(path, hparams, tensors, primary_type=0, bundles=None, n_ctx_train=2048):
    """tensors: [(name, qtype, shape (GGUF order, ne0 first), data bytes,
    layer_index, hot)] in file order; hot tensors go to the hot region, the
    others to their layer's cold region.  bundles: None, or (bundle_size,
    n_ff, [per-layer list of bundle byte strings]) for a version-2 file.
    Returns the header dict."""
    n_layers = hparams["n_layers"]
    hot = [t for t in tensors if t[5]]
    cold = [[t for t in tensors if not t[5] and t[4] == L] for L in range(n_layers)]
    ordered = hot + [t for L in range(n_layers) for t in cold[L]]
    index_size = n_layers * LAYER_BYTES + len(ordered) * ENTRY_BYTES
    h = dict(magic=MAGIC, version=1, n_layers=n_layers, n_tensors=len(ordered),
             index_offset=HEADER_BYTES, index_size=index_size,
             hot_offset=align4k(HEADER_BYTES + index_size),
             hot_size=sum(align4k(len(t[3])) for t in hot),
             n_embd=hparams["n_embd"], n_heads=hparams["n_heads"],
             n_heads_kv=hparams["n_heads_kv"], n_ff=hparams["n_ff"],
             n_vocab=hparams["n_vocab"], n_ctx_train=n_ctx_train,
             rope_freq_base=hparams["rope_freq_base"], rms_norm_eps=hparams["rms_norm_eps"],
             primary_type=primary_type, bundle_index_offset=0)
    h["cold_start_offset"] = align4k(h["hot_offset"] + h["hot_size"])
    entries, layer_descs, body = [], [], {}
    cur = 0
    for t in hot:
        entries.append(entry_bytes(t[0], t[1], t[2], len(t[2]), cur, len(t[3]), t[4], 1))
        body[h["hot_offset"] + cur] = t[3]
        cur += align4k(len(t[3]))
    cursor = h["cold_start_offset"]
    for L in range(n_layers):
        start, off = align4k(cursor), 0
        for t in cold[L]:
            entries.append(entry_bytes(t[0], t[1], t[2], len(t[2]), off, len(t[3]), L, 0))
            body[start + off] = t[3]
            off += align4k(len(t[3]))
        layer_descs.append(struct.pack("<QQII", start, off, len(cold[L]), 0))
        cursor = start + off
    h["cold_total_size"] = cursor - h["cold_start_offset"]
    end = align4k(cursor)
    bundle_index = b""
    if bundles is not None:
        size, n_ff, per_layer = bundles
        descs = []
        for blist in per_layer:
            if not blist:
                descs.append(struct.pack("<QQII", 0, 0, 0, 0))
                continue
            descs.append(struct.pack("<QQII", end, n_ff * size, n_ff, size))
            for j, bb in enumerate(blist):
                body[end + j * size] = bb
            end += n_ff * size
        end = align4k(end)
        h["bundle_index_offset"] = end
        h["version"] = 2
        bundle_index = struct.pack("<IIII", len(per_layer), size, n_ff, 0) + b"".join(descs)
    out = bytearray(end + len(bundle_index))
    out[:HEADER_BYTES] = header_bytes(h)
    idx = b"".join(layer_descs) + b"".join(entries)
    out[HEADER_BYTES:HEADER_BYTES + len(idx)] = idx
    for off, data in body.items():
        out[off:off + len(data)] = data
    out[end:] = bundle_index
    with open(path, "wb") as f:
        f.write(out)
    return h
