"""INT8 checkpoint loading for the W8A8 projections (the reference's
rank_local_int8 plan / load, on one GPU).

The checkpoint format is the reference's Native INT8 ConvRot layout
(patches/rank_local_int8.py:37-114): per projection a safetensors ``weight``
(I8 [N, K]), ``weight_scale`` (F32 [N, 1]) and ``comfy_quant`` (U8 bytes of
the JSON {"format": "int8_tensorwise", "convrot": true,
"convrot_groupsize": 256}). A block's projections are loaded straight into
this package's ColumnParallelLinearINT8 / RowParallelLinearINT8 modules; with
``world_size`` 2 each rank reads its component-wise column rows or its K
half (which must keep whole 256-channel ConvRot groups), so a rank's half of
a layer is read without materializing the whole tensor. Tensors are read
through safetensors' memory map, row/column ranges only.
"""
import json
from pathlib import Path

import torch
from torch import nn

from .tp_dit import ColumnParallelLinearINT8, RowParallelLinearINT8

QUANT_CONFIG = {'format': 'int8_tensorwise', 'convrot': True, 'convrot_groupsize': 256}

# Projections of a block: name -> (checkpoint path under the block prefix,
# packed column components, or 0 for a row-parallel projection).
DIT_LINEARS = {'qkv_proj': ('attn.qkv_proj', 3), 'out_proj': ('attn.out_proj', 0),
               'fc1': ('mlp.fc1', 2), 'fc2': ('mlp.fc2', 0)}
TE_LINEARS = {n: (('self_attn.' if n in ('q_proj', 'k_proj', 'v_proj', 'o_proj') else 'mlp.') + n,
                  0 if n in ('o_proj', 'down_proj') else 1)
              for n in ('q_proj', 'k_proj', 'v_proj', 'o_proj', 'gate_proj', 'up_proj', 'down_proj')}
DIT_REPLICATED = dict({n + '.weight': ('attn.' if n in ('q_norm', 'k_norm') else '') + n + '.weight'
                       for n in ('norm1', 'norm2', 'q_norm', 'k_norm')},
                      **{'adaln_proj.' + n: 'adaln_proj.linear.' + n for n in ('weight', 'bias')})
TE_REPLICATED = {n + '.weight': ('self_attn.' if n in ('q_norm', 'k_norm') else '') + n + '.weight'
                 for n in ('input_layernorm', 'post_attention_layernorm', 'q_norm', 'k_norm')}


class CheckpointReader:
    """Header and ranged reads of one safetensors file (memory-mapped).

    ``header[name]`` is the safetensors entry ({'dtype', 'shape', ...});
    ``read_tensor(name, rows=None, columns=None)`` reads a list of row ranges
    [(a, b), ...] and/or one column range (a, b) of a 2-D tensor.
    """

    def __init__(self, path):
        from safetensors import safe_open
        self.path = Path(path)
        with open(self.path, 'rb') as f:
            n = int.from_bytes(f.read(8), 'little')
            header = json.loads(f.read(n))
        header.pop('__metadata__', None)
        self.header = header
        self._file = safe_open(str(self.path), framework='pt', device='cpu')

    def read_tensor(self, name, rows=None, columns=None):
        if name not in self.header:
            raise KeyError(name)
        sl = self._file.get_slice(name)
        if rows is None and columns is None:
            return self._file.get_tensor(name)
        cols = slice(None) if columns is None else slice(columns[0], columns[1])
        ranges = [(0, self.header[name]['shape'][0])] if rows is None else rows
        parts = [sl[a:b, cols] for a, b in ranges]
        return parts[0] if len(parts) == 1 else torch.cat(parts, 0)


def plan(reader, kind, index, rank=0, world_size=1):
    """(target, source, rows, columns) reads of one block's rank part.

    Follows patches/rank_local_int8.py:37-91: component-wise packed rows for
    column projections (``components`` equal chunks, each split in
    ``world_size`` contiguous parts), K halves for row projections (K must
    divide into whole 256-channel ConvRot groups per rank), replicated norms
    and AdaLN tensors (all required). Raises ValueError on a dtype, shape or
    metadata name the layout does not allow, on a missing tensor, on shapes
    that do not form one block geometry, and on tensors under the block
    prefix that the layout does not know.
    """
    if world_size not in (1, 2) or not 0 <= rank < world_size:
        raise ValueError('world_size 1 or 2 and a rank below it required')
    if kind == 'dit':
        prefix, linears, replicated = f'blocks.{index}.', DIT_LINEARS, DIT_REPLICATED
    elif kind == 'te':
        prefix, linears, replicated = f'model.layers.{index}.', TE_LINEARS, TE_REPLICATED
    else:
        raise ValueError('Only TE and DiT blocks are supported')
    result, known = [], set()
    for target, source in replicated.items():
        if prefix + source not in reader.header:
            raise ValueError('Missing replicated block tensor: ' + prefix + source)
        result.append((target, prefix + source, None, None))
        known.add(prefix + source)
    quant_names = []
    for target, (source, components) in linears.items():
        for suffix in ('weight', 'weight_scale'):
            name = prefix + source + '.' + suffix
            if name not in reader.header:
                raise ValueError('Missing INT8 projection tensor: ' + name)
            info = reader.header[name]
            if info['dtype'] != ('I8' if suffix == 'weight' else 'F32'):
                raise ValueError('Unsupported Native quantization dtype: ' + name)
            shape = info['shape']
            if len(shape) != 2 or (suffix == 'weight_scale' and shape[1] != 1):
                raise ValueError('Unsupported Native quantization shape: ' + name)
            rows = columns = None
            if components:
                full = shape[0]
                if full % (world_size * components):
                    raise ValueError('Invalid packed component shape: ' + name)
                chunk = full // components
                rows = [(i * chunk + rank * chunk // world_size, i * chunk + (rank + 1) * chunk // world_size)
                        for i in range(components)]
            elif suffix == 'weight':
                width = shape[1]
                if width % (256 * world_size):
                    raise ValueError('Row shard must preserve 256-channel ConvRot groups: ' + name)
                columns = (rank * width // world_size, (rank + 1) * width // world_size)
            result.append((target + '.' + suffix, name, rows, columns))
            known.add(name)
        qname = prefix + source + '.comfy_quant'
        if qname not in reader.header:
            raise ValueError('Missing quantization metadata: ' + qname)
        known.add(qname)
        quant_names.append(qname)
    unexpected = {n for n in reader.header if n.startswith(prefix)} - known
    if unexpected:
        raise ValueError('Unqualified Native block metadata/tensors: ' + str(sorted(unexpected)))
    _check_geometry(reader, kind, prefix, linears, replicated)
    return result, quant_names


def _check_geometry(reader, kind, prefix, linears, replicated):
    """The block's tensors must agree with one transformer geometry (the
    reference checks them against its TP module shells,
    patches/rank_local_int8.py:84-90): hidden size from the first column
    projection's K, 128-wide heads, FFN widths that pair up."""
    def shape(target):
        if target in linears:
            return reader.header[prefix + linears[target][0] + '.weight']['shape']
        return reader.header[prefix + replicated[target]]['shape']

    def need(ok, target):
        if not ok:
            name = prefix + (linears[target][0] + '.weight' if target in linears else replicated[target])
            raise ValueError('Checkpoint shape differs from Native TP configuration: ' + name)

    head = 128
    if kind == 'dit':
        hidden = shape('qkv_proj')[1]
        inner = shape('out_proj')[1]
        need(shape('qkv_proj')[0] == 3 * inner and inner % head == 0, 'qkv_proj')
        need(shape('out_proj')[0] == hidden, 'out_proj')
        need(shape('fc1')[1] == hidden and shape('fc1')[0] % 2 == 0, 'fc1')
        need(shape('fc2') == [hidden, shape('fc1')[0] // 2], 'fc2')
        for n in ('norm1.weight', 'norm2.weight'):
            need(shape(n) == [hidden], n)
        for n in ('q_norm.weight', 'k_norm.weight'):
            need(shape(n) == [head], n)
        w, b = shape('adaln_proj.weight'), shape('adaln_proj.bias')
        need(len(w) == 2 and w[0] == 18 * hidden, 'adaln_proj.weight')
        need(b == [18 * hidden], 'adaln_proj.bias')
    else:
        hidden = shape('q_proj')[1]
        for n in ('q_proj', 'k_proj', 'v_proj', 'gate_proj', 'up_proj'):
            need(shape(n)[1] == hidden and shape(n)[0] % head == 0, n)
        need(shape('k_proj')[0] == shape('v_proj')[0], 'v_proj')
        need(shape('o_proj') == [hidden, shape('q_proj')[0]], 'o_proj')
        need(shape('up_proj')[0] == shape('gate_proj')[0], 'up_proj')
        need(shape('down_proj') == [hidden, shape('gate_proj')[0]], 'down_proj')
        for n in ('input_layernorm.weight', 'post_attention_layernorm.weight'):
            need(shape(n) == [hidden], n)
        for n in ('q_norm.weight', 'k_norm.weight'):
            need(shape(n) == [head], n)


class INT8Block(nn.Module):
    """One block's INT8 projections (this package's modules) and its
    replicated tensors (norm gains, AdaLN projection) as buffers."""

    def __init__(self, kind, projections, replicated, metadata):
        super().__init__()
        self.kind = kind
        for name, module in projections.items():
            setattr(self, name, module)
        self.projection_names = tuple(projections)
        self.replicated = {}
        for name, t in replicated.items():
            self.register_buffer(name.replace('.', '_'), t)
            self.replicated[name] = name.replace('.', '_')
        self._rank_checkpoint_metadata = metadata

    def tensor(self, name):
        return getattr(self, self.replicated[name])


def load_block(source, kind, index, *, rank=0, world_size=1, device=None):
    """Load one DiT or TE block's INT8 projections into W8A8 modules.

    patches/rank_local_int8.py:98-114 (load_rank_block) on this package's
    modules: validates the quantization metadata of every projection, reads
    only the rank's rows/columns, and returns an INT8Block whose projections
    carry ``weight`` int8 [N, K_rank] and ``weight_scale`` fp32 [N, 1] on
    ``device``.
    """
    reader = source if isinstance(source, CheckpointReader) else CheckpointReader(source)
    device = torch.device(device) if device is not None else torch.device('cuda', 0)
    mappings, quant_names = plan(reader, kind, index, rank, world_size)
    metadata = {}
    for name in quant_names:
        raw = reader.read_tensor(name)
        config = json.loads(bytes(raw.to(torch.uint8).tolist()).decode('utf8'))
        if config != QUANT_CONFIG:
            raise ValueError('Unqualified quantization metadata: ' + str(config))
        metadata[name] = config
    linears = DIT_LINEARS if kind == 'dit' else TE_LINEARS
    tensors = {target: reader.read_tensor(name, rows=rows, columns=columns)
               for target, name, rows, columns in mappings}
    projections = {}
    for target, (_, components) in linears.items():
        w = tensors[target + '.weight']
        s = tensors[target + '.weight_scale']
        n, k = w.shape
        if components:
            m = ColumnParallelLinearINT8(k, n, device=device, components=components)
        else:
            m = RowParallelLinearINT8(k, n, device=device)
        if s.shape[0] != n:
            raise ValueError('Weight scale rows differ from weight rows: ' + target)
        m.world_size = world_size
        m.rank = rank
        m.weight.data.copy_(w)
        m.weight_scale.data.copy_(s)
        projections[target] = m
    # Replicated tensors take the dtype of the reference's module shells
    # (patches/rank_local_int8.py:12-15,108-109): FP32 for the DiT, FP16 for
    # the text encoder.
    dtype = torch.float32 if kind == 'dit' else torch.float16
    replicated = {t: tensors[t].to(device=device, dtype=dtype) for t in tensors if not t.split('.')[0] in linears}
    return INT8Block(kind, projections, replicated, metadata).eval().requires_grad_(False)


def save_block(path, kind, index, weights, replicated=None):
    """Write a block in the Native INT8 layout (used to make fixtures).

    weights: {projection: (int8 [N, K], fp32 [N, 1])} under this module's
    projection names; replicated: {target name: tensor} (norm gains, AdaLN).
    """
    from safetensors.torch import save_file
    if kind == 'dit':
        prefix, linears, rep = f'blocks.{index}.', DIT_LINEARS, DIT_REPLICATED
    else:
        prefix, linears, rep = f'model.layers.{index}.', TE_LINEARS, TE_REPLICATED
    out = {}
    blob = torch.tensor(list(json.dumps(QUANT_CONFIG).encode('utf8')), dtype=torch.uint8)
    for target, (w, s) in weights.items():
        source = linears[target][0]
        out[prefix + source + '.weight'] = w.to(torch.int8).contiguous()
        out[prefix + source + '.weight_scale'] = s.to(torch.float32).reshape(-1, 1).contiguous()
        out[prefix + source + '.comfy_quant'] = blob.clone()
    for target, t in (replicated or {}).items():
        out[prefix + rep[target]] = t.contiguous()
    save_file(out, str(path))
    return Path(path)
