'use strict';
/**
 * Node host for libqlinear: the reference's TypeScript surface for the GPTQ int4 path, with the
 * int4 work on the MI355X through the Node-API addon (webllm_amd/lib/qlinear_napi.node).
 *
 * Same names, argument meaning and error behaviour as (paths in the intplusplus/webllm checkout):
 *   parseSafetensors, parseSafetensorsHeader,    src/weights/safetensors.ts:40-222
 *   requireTensor, expectTensor, tensorCount,
 *   readTensorBytes, readTensorF32, f16BitsToF32,
 *   dtypeByteSize
 *   dequantizeGptqInt4(params)                   src/weights/quant.ts:42-118 (exact, on the GPU)
 *   QuantLinearModel.gemm(A, weight, C, bias,    src/model/qwen.ts:568-618 QwenGpt.gemm
 *     M, N, K)
 *   loadQwenWeights(ctx, model, options)         src/weights/qwen-loader.ts:102-177 (async), with
 *                                                the packed int4 tensors uploaded as they are
 *   readF16Rows                                  src/weights/qwen-loader.ts:70-93
 *   checkGIdx, countStoredZeros                  src/tests/qwen/qwen-format.ts:112-130 probes
 *   QWEN25_05B, qwenKvDim                        src/model/qwen-config.ts:1-54
 *
 * Errors are thrown as Error (the reference's `throw new Error(msg)`); library status codes carry
 * `err.code` = 'QL_E_*'. There is no CPU fallback: a missing addon throws at require time.
 */
const fs = require('fs');
const path = require('path');

const ADDON_PATH = path.join(__dirname, '..', 'lib', 'qlinear_napi.node');
if (!fs.existsSync(ADDON_PATH)) {
    throw new Error(`qlinear: addon not built at ${ADDON_PATH} (run __graft_entry__.build())`);
}
const addon = require(ADDON_PATH);

const QL_DTYPE_F32 = 0;
const QL_DTYPE_F16 = 1;

// ------------------------------------------------------------------ config (qwen-config.ts)

const QWEN25_05B = Object.freeze({
    vocabSize: 151936, blockSize: 128, nLayer: 24, nHead: 14, nKvHead: 2, nEmbd: 896,
    intermediate: 4864, rmsEps: 1e-6, ropeTheta: 1000000,
});

function qwenHeadDim(c) { return c.nEmbd / c.nHead; }
function qwenKvDim(c) { return c.nKvHead * qwenHeadDim(c); }

// ------------------------------------------------------------------ safetensors.ts

const DTYPE_BYTES = { F64: 8, I64: 8, F32: 4, I32: 4, F16: 2, BF16: 2, I16: 2, I8: 1, U8: 1, BOOL: 1 };

function dtypeByteSize(dtype) {
    const n = DTYPE_BYTES[dtype];
    if (n === undefined) throw new Error(`unknown safetensors dtype: ${dtype}`);
    return n;
}

function parseSafetensorsHeader(headerBytes) {
    let parsed;
    try {
        parsed = JSON.parse(Buffer.from(headerBytes.buffer, headerBytes.byteOffset,
            headerBytes.byteLength).toString('utf8'));
    } catch (err) {
        throw new Error(`safetensors: header JSON parse failed: ${err.message}`);
    }
    if (typeof parsed !== 'object' || parsed === null) {
        throw new Error('safetensors: header is not a JSON object');
    }
    const header = {};
    for (const name of Object.keys(parsed)) {
        if (name === '__metadata__') continue;
        const item = parsed[name];
        if (typeof item !== 'object' || item === null) throw new Error(`safetensors: ${name} entry invalid`);
        if (typeof item.dtype !== 'string') throw new Error(`safetensors: ${name} missing dtype`);
        if (!Array.isArray(item.shape)) throw new Error(`safetensors: ${name} missing shape`);
        if (!Array.isArray(item.data_offsets) || item.data_offsets.length !== 2) {
            throw new Error(`safetensors: ${name} data_offsets invalid`);
        }
        const start = Number(item.data_offsets[0]);
        const end = Number(item.data_offsets[1]);
        if (!Number.isFinite(start) || !Number.isFinite(end) || start < 0 || end < start) {
            throw new Error(`safetensors: ${name} data_offsets out of range`);
        }
        header[name] = { dtype: item.dtype, shape: item.shape.map(Number), data_offsets: [start, end] };
    }
    return header;
}

/** buffer: ArrayBuffer or Node Buffer / Uint8Array (the whole file). */
function parseSafetensors(buffer) {
    const bytes = buffer instanceof ArrayBuffer ? new Uint8Array(buffer)
        : new Uint8Array(buffer.buffer, buffer.byteOffset, buffer.byteLength);
    if (bytes.byteLength < 8) throw new Error('safetensors: buffer too short');
    const dv = new DataView(bytes.buffer, bytes.byteOffset, bytes.byteLength);
    const headerLen = dv.getUint32(0, true);
    if (dv.getUint32(4, true) !== 0) throw new Error('safetensors: header longer than 4 GiB is not supported');
    const dataStart = 8 + headerLen;
    if (headerLen <= 0 || dataStart > bytes.byteLength) {
        throw new Error(`safetensors: invalid header length headerLen=${headerLen} bufferSize=${bytes.byteLength}`);
    }
    const header = parseSafetensorsHeader(bytes.subarray(8, dataStart));
    for (const name of Object.keys(header)) {
        if (dataStart + header[name].data_offsets[1] > bytes.byteLength) {
            throw new Error(`safetensors: ${name} data out of bounds end=${header[name].data_offsets[1]}`);
        }
    }
    return { buffer: bytes, dataStart, header };
}

function tensorCount(entry) { return entry.shape.reduce((a, b) => a * b, 1); }

function requireTensor(file, name) {
    const entry = file.header[name];
    if (!entry) throw new Error(`safetensors: missing tensor ${name}`);
    return entry;
}

function expectTensor(file, name, dtype, shape) {
    const entry = requireTensor(file, name);
    if (entry.dtype !== dtype) throw new Error(`safetensors: ${name} dtype=${entry.dtype}, expected ${dtype}`);
    if (entry.shape.length !== shape.length || entry.shape.some((v, i) => v !== shape[i])) {
        throw new Error(`safetensors: ${name} shape=[${entry.shape}], expected [${shape}]`);
    }
    return entry;
}

function f16BitsToF32(bits) {
    const sign = (bits & 0x8000) !== 0 ? -1 : 1;
    const exp = (bits >>> 10) & 0x1f;
    const mant = bits & 0x03ff;
    if (exp === 0) return sign * mant * Math.pow(2, -24);
    if (exp === 31) return mant === 0 ? sign * Infinity : NaN;
    return sign * (1 + mant / 1024) * Math.pow(2, exp - 15);
}

/** Raw bytes of one tensor, as a copy (aligned for typed views). */
function readTensorBytes(file, name) {
    const entry = requireTensor(file, name);
    const start = file.dataStart + entry.data_offsets[0];
    const length = tensorCount(entry) * dtypeByteSize(entry.dtype);
    return Uint8Array.from(file.buffer.subarray(start, start + length));
}

function readTensorF32(file, name) {
    const entry = requireTensor(file, name);
    const count = tensorCount(entry);
    const start = file.dataStart + entry.data_offsets[0];
    const view = new DataView(file.buffer.buffer, file.buffer.byteOffset + start,
        entry.data_offsets[1] - entry.data_offsets[0]);
    const out = new Float32Array(count);
    const tmp = new DataView(new ArrayBuffer(4));
    for (let i = 0; i < count; i++) {
        switch (entry.dtype) {
            case 'F32': out[i] = view.getFloat32(i * 4, true); break;
            case 'F16': out[i] = f16BitsToF32(view.getUint16(i * 2, true)); break;
            case 'BF16':
                tmp.setUint32(0, view.getUint16(i * 2, true) << 16, true);
                out[i] = tmp.getFloat32(0, true);
                break;
            case 'U8': out[i] = view.getUint8(i); break;
            case 'I8': out[i] = view.getInt8(i); break;
            default: throw new Error(`readTensorF32: unsupported dtype ${entry.dtype} (${name})`);
        }
    }
    return out;
}

// ------------------------------------------------------------------ device objects

/** Bump allocator over one arena, 256-byte aligned slices (the library's alignment contract). */
class ArenaLayout {
    constructor() { this.used = 0; }
    take(nbytes, align) {
        const a = align || 256;
        const off = Math.ceil(this.used / a) * a;
        this.used = off + nbytes;
        return off;
    }
}

class Arena {
    constructor(ctx, bytes) {
        this.ctx = ctx;
        this.handle = addon.arenaReserve(ctx.handle, bytes);
        this.size = bytes;
        ctx._arenas.add(this);
    }
    write(off, typed) { addon.arenaWrite(this.handle, off, typed); }
    read(off, typed) { addon.arenaRead(this.handle, off, typed); return typed; }
    release() {
        if (this.handle) {
            addon.arenaRelease(this.handle);
            this.handle = null;
            this.ctx._arenas.delete(this);
        }
    }
}

/**
 * A forward's decode linears as one persistent launch (ql_seq_*; the CommandBatch of
 * src/gpu/pipeline.ts:71-116 with passBreak, qwen.ts:556-559): linear i consumes linear j's
 * output when xOffs[i] === yOffs[j], and the kernel orders the two on the device.
 * `fuse` (optional, one entry per linear, null for none) folds the layer's elementwise work in
 * (ql_seq_create_fused; qwen.ts:401-405, :445-478): {normWOff, normEps} normalizes the linear's
 * input (RMSNorm weights at normWOff in `weights`), {x2Off} multiplies silu(x) by a second input,
 * {resOff} adds a residual to the output. An offset equal to another linear's yOffs entry makes
 * that linear the producer.
 */
class Seq {
    constructor(ctx, descs, weights, act, xOffs, xDtype, M, yOffs, fuse) {
        this.ctx = ctx;
        this.handle = fuse
            ? addon.seqCreate(ctx.handle, descs, weights.handle, act.handle, xOffs, xDtype, M, yOffs, fuse)
            : addon.seqCreate(ctx.handle, descs, weights.handle, act.handle, xOffs, xDtype, M, yOffs);
        ctx._seqs.add(this);
    }
    get info() { return addon.seqInfo(this.handle); }
    run() { addon.seqRun(this.ctx.handle, this.handle); }
    /** Waits for the stream; throws QL_E_STATE if a run was aborted. */
    status() { addon.seqStatus(this.ctx.handle, this.handle); }
    destroy() {
        if (this.handle) {
            addon.seqDestroy(this.handle);
            this.handle = null;
            this.ctx._seqs.delete(this);
        }
    }
}

/** One device, one stream (ql_create). */
class Context {
    constructor(device) {
        this.handle = addon.create(device === undefined ? 0 : device);
        this._arenas = new Set();
        this._seqs = new Set();
    }
    seq(descs, weights, act, xOffs, xDtype, M, yOffs, fuse) {
        return new Seq(this, descs, weights, act, xOffs, xDtype, M, yOffs, fuse);
    }
    info() { return addon.deviceInfo(this.handle); }
    arena(bytes) { return new Arena(this, bytes); }
    sync() { addon.sync(this.handle); }
    timerStart() { addon.timerStart(this.handle); }
    timerStop() { return addon.timerStop(this.handle); }
    destroy() {
        for (const q of Array.from(this._seqs)) q.destroy();
        for (const a of Array.from(this._arenas)) a.release();
        if (this.handle) { addon.destroy(this.handle); this.handle = null; }
    }
}

function makeDesc(qweightOff, qzerosOff, scalesOff, K, N, group, biasOff, bits) {
    return {
        qweightOff, qzerosOff: qzerosOff === undefined ? null : qzerosOff, scalesOff,
        biasOff: biasOff === undefined ? null : biasOff, K, N,
        group: group === undefined ? 128 : group, bits: bits === undefined ? 4 : bits,
    };
}

const CODE_NAMES = {
    '-1': 'QL_E_BITS', '-2': 'QL_E_GROUP', '-3': 'QL_E_DIMS', '-4': 'QL_E_QWEIGHT_SHORT',
    '-5': 'QL_E_SCALES_SHORT', '-6': 'QL_E_QZEROS_SHORT', '-7': 'QL_E_GROUP_PACK',
};

function libError(code, message) {
    const e = new Error(`${code}: ${message}`);
    e.code = code;
    return e;
}

// ------------------------------------------------------------------ quant.ts

let defaultCtx = null;

/**
 * quant.ts:42-118: GptqInt4Params -> fp32 [outFeatures, inFeatures], computed on the GPU
 * (ql_unpack_f32_ex with the f32 scales as given: any Float32Array, quant.ts:22-23; bit-identical
 * to the reference's loop). `ctx` defaults to device 0.
 */
function dequantizeGptqInt4(params, ctx) {
    const groupSize = params.groupSize === undefined || params.groupSize === null ? 128 : params.groupSize;
    const bits = params.bits === undefined || params.bits === null ? 4 : params.bits;
    const inF = params.inFeatures;
    const outF = params.outFeatures;
    // quant.ts:46-79 order: bits, group, dims, qweight bytes, scales count, qzeros bytes, group % 8
    const shapeRc = addon.validate(makeDesc(0, null, 0, inF, outF, groupSize, null, bits), 2 ** 52);
    if (shapeRc === -1 || shapeRc === -2 || shapeRc === -3) throw libError(CODE_NAMES[shapeRc], addon.lastError());
    const need = addon.gptqSizes(inF, outF, groupSize);
    if (params.qweight.byteLength < need.qweightBytes) {
        throw libError('QL_E_QWEIGHT_SHORT', `GPTQ: qweight needs ${need.qweightBytes} bytes, got ${params.qweight.byteLength}`);
    }
    if (params.scales.length < need.scalesBytes / 2) {
        throw libError('QL_E_SCALES_SHORT', `GPTQ: scales need ${need.scalesBytes / 2} values, got ${params.scales.length}`);
    }
    const qz = params.qzeros || null;
    if (qz && qz.byteLength < need.qzerosBytes) {
        throw libError('QL_E_QZEROS_SHORT', `GPTQ: qzeros need ${need.qzerosBytes} bytes, got ${qz.byteLength}`);
    }
    if (shapeRc === -7) throw libError('QL_E_GROUP_PACK', `GPTQ: groupSize=${groupSize} must be a multiple of 8`);
    const s32 = Float32Array.from(params.scales.subarray(0, need.scalesBytes / 2));
    if (!ctx) { if (!defaultCtx) defaultCtx = new Context(0); ctx = defaultCtx; }
    const lay = new ArenaLayout();
    const oQw = lay.take(need.qweightBytes);
    const oQz = qz ? lay.take(need.qzerosBytes) : null;
    const oSc = lay.take(s32.byteLength);
    const w = ctx.arena(lay.used + 256);
    const out = ctx.arena(Math.max(inF * outF * 4, 16));
    try {
        w.write(oQw, params.qweight.subarray(0, need.qweightBytes));
        if (qz) w.write(oQz, qz.subarray(0, need.qzerosBytes));
        w.write(oSc, s32);
        addon.unpack(ctx.handle, makeDesc(oQw, oQz, oSc, inF, outF, groupSize, null, bits), w.handle,
            out.handle, 0, true, QL_DTYPE_F32);
        return out.read(0, new Float32Array(outF * inF));
    } finally {
        w.release();
        out.release();
    }
}

// ------------------------------------------------------------------ QwenGpt weight side (qwen.ts)

/** Slice of a device arena: {arena, offset, length, shape, dtype} (buffer.ts:12-18). */
class Tensor {
    constructor(arena, offset, length, shape, dtype, pool) {
        this.arena = arena; this.offset = offset; this.length = length; this.shape = shape;
        this.dtype = dtype; this.pool = pool || null;
    }
    read() {
        const T = this.dtype === 'f16' ? Uint16Array : (this.dtype === 'u32' ? Uint32Array : Float32Array);
        return this.arena.read(this.offset, new T(this.length));
    }
    write(data) { this.arena.write(this.offset, data); }
}

/** Per-step activation arena (arena.ts): bump allocation from the front, split-K scratch from the back. */
class ActivationArena {
    constructor(ctx, bytes) {
        this.arena = ctx.arena(bytes);
        this.layout = new ArenaLayout();
    }
    alloc(shape, dtype) {
        const dt = dtype || 'f32';
        const n = shape.reduce((a, b) => a * b, 1);
        const off = this.layout.take(n * (dt === 'f16' ? 2 : 4));
        if (this.layout.used > this.arena.size) throw new Error('activation arena exhausted');
        return new Tensor(this.arena, off, n, shape.slice(), dt, this);
    }
    scratchOffset(nbytes) {
        const off = Math.floor((this.arena.size - nbytes) / 256) * 256;
        if (off < this.layout.used) throw new Error(`activation arena: no room for ${nbytes} scratch bytes`);
        return off;
    }
    reset() { this.layout = new ArenaLayout(); }
    release() { this.arena.release(); }
}

class QuantLinearModel {
    /** Weight side of QwenGpt with GPTQ weights kept packed in one device arena, addressed by name. */
    constructor(ctx, weightCapacity) {
        this.ctx = ctx;
        this.weights = ctx.arena(weightCapacity);
        this.layout = new ArenaLayout();
        this.linears = new Map();
        this.f32Weights = new Map();
        this.f16Weights = new Map();
    }
    get weightBytes() { return this.layout.used; }
    _place(typed) {
        const off = this.layout.take(typed.byteLength);
        if (this.layout.used > this.weights.size) {
            throw new Error(`weight arena exhausted (${this.layout.used} > ${this.weights.size})`);
        }
        this.weights.write(off, typed);
        return off;
    }
    /** qweight I32 [in/8, out], qzeros I32 [in/g, out/8] or null, scales F16 bits [in/g, out], bias F32 [out] or null. */
    uploadGptqLinear(name, p) {
        if (this.linears.has(name)) throw new Error(`weight already exists: ${name}`);
        const group = p.groupSize || 128;
        const qw = this._place(p.qweight);
        const qz = p.qzeros ? this._place(p.qzeros) : null;
        const sc = this._place(p.scalesF16);
        const b = p.bias ? this._place(Float32Array.from(p.bias)) : null;
        const desc = makeDesc(qw, qz, sc, p.inFeatures, p.outFeatures, group, b);
        const rc = addon.validate(desc, this.weights.size);
        if (rc !== 0) throw libError(CODE_NAMES[rc] || 'QL_E_INVALID', addon.lastError());
        this.linears.set(name, { desc, K: p.inFeatures, N: p.outFeatures });
    }
    uploadF32(name, data) {
        if (this.f32Weights.has(name)) throw new Error(`weight already exists: ${name}`);
        const a = Float32Array.from(data);
        this.f32Weights.set(name, new Tensor(this.weights, this._place(a), a.length, [a.length], 'f32'));
    }
    uploadF16Bits(name, bytes, shape) {
        if (this.f16Weights.has(name)) throw new Error(`weight already exists: ${name}`);
        const n = shape.reduce((x, y) => x * y, 1);
        this.f16Weights.set(name, new Tensor(this.weights, this._place(bytes), n, shape.slice(), 'f16'));
    }
    linear(name) {
        const l = this.linears.get(name);
        if (!l) throw new Error(`missing int4 weight: ${name}`);
        return l;
    }
    /** C[M,N] = A[M,K] @ W^T (+ bias) — qwen.ts:568-618. A f32 or f16, C f32. */
    gemm(A, weight, C, bias, M, N, K) {
        if (this.f16Weights.has(weight) && !this.linears.has(weight)) return this._gemmF16(A, weight, C, bias, M, N, K);
        const lin = this.linear(weight);
        if (lin.K !== K || lin.N !== N) throw new Error(`gemm: ${weight} is [${lin.N},${lin.K}], called with N=${N} K=${K}`);
        if (bias !== null && bias !== undefined && lin.desc.biasOff === null) throw new Error(`missing f32 weight: ${bias}`);
        let desc = lin.desc;
        if ((bias === null || bias === undefined) && desc.biasOff !== null) desc = Object.assign({}, desc, { biasOff: null });
        if (A.arena !== C.arena || !A.pool || A.pool !== C.pool) throw new Error('gemm: A and C must come from one ActivationArena');
        if (A.length < M * K || C.length < M * N) throw new Error('gemm: tensor too small for [M,K] / [M,N]');
        const plan = addon.planLinear(M, N, K, desc.group);
        const scratch = A.pool.scratchOffset(plan.scratchBytes);
        addon.linear(this.ctx.handle, desc, this.weights.handle, A.arena.handle, A.offset,
            A.dtype === 'f16' ? QL_DTYPE_F16 : QL_DTYPE_F32, M, C.offset, scratch);
    }
    /** fp16 weights (the tied lm_head `embed`, qwen.ts:488-489): f32 A and C, fp32 accumulation. */
    _gemmF16(A, weight, C, bias, M, N, K) {
        const w = this.f16Weights.get(weight);
        if (w.shape[0] !== N || w.shape[1] !== K) throw new Error(`gemm: ${weight} is [${w.shape}], called with N=${N} K=${K}`);
        let b = null;
        if (bias !== null && bias !== undefined) {
            const t = this.f32Weights.get(bias);
            if (!t) throw new Error(`missing f32 weight: ${bias}`);
            b = t.offset;
        }
        if (A.dtype !== 'f32' || C.dtype !== 'f32') throw new Error('gemm over fp16 weights takes f32 A and C');
        if (A.arena !== C.arena) throw new Error('gemm: A and C must live in the same activation arena');
        if (A.length < M * K || C.length < M * N) throw new Error('gemm: tensor too small for [M,K] / [M,N]');
        addon.gemvF16w(this.ctx.handle, this.weights.handle, w.offset, b, A.arena.handle, A.offset, M, N, K, C.offset);
    }
    /** out[M, C] = rows tokens[0..M) of the fp16 table as f32 (embedding_f16.wgsl, qwen.ts:391-392);
     *  token ids >= vocab give zero rows. */
    embed(tokens, out, M, weight) {
        const name = weight || 'embed';
        const w = this.f16Weights.get(name);
        if (!w) throw new Error(`missing f16 weight: ${name}`);
        const vocab = w.shape[0], C = w.shape[1];
        if (tokens.dtype !== 'u32' || tokens.length < M) throw new Error('embed: tokens must be a u32 tensor of at least M ids');
        if (out.dtype !== 'f32' || out.length < M * C || out.arena !== tokens.arena)
            throw new Error("embed: out must be an f32 [M, C] tensor in the tokens' arena");
        addon.embedF16(this.ctx.handle, this.weights.handle, w.offset, vocab, C, tokens.arena.handle, tokens.offset, M, out.offset);
    }
    /** y = rmsnorm(x (+ residual)) * weight; the sum goes to sumOut (vec_add + rmsnorm.wgsl in one launch). */
    rmsnorm(x, weight, y, M, C, eps, residual, sumOut) {
        const w = this.f32Weights.get(weight);
        if (!w) throw new Error(`missing f32 weight: ${weight}`);
        if (w.length !== C) throw new Error(`rmsnorm: ${weight} has ${w.length} values, C=${C}`);
        for (const t of [y, residual, sumOut]) {
            if (t && t.arena !== x.arena) throw new Error('rmsnorm: x, y, residual and sumOut must share one arena');
        }
        addon.addRmsNorm(this.ctx.handle, x.arena.handle, x.offset, residual ? residual.offset : null,
            this.weights.handle, w.offset, eps, M, C, sumOut ? sumOut.offset : null, y.offset);
    }
    /** out = silu(gate) * up (silu_mul.wgsl, qwen.ts:468-469). */
    siluMul(gate, up, out, n) {
        if (gate.arena !== up.arena || gate.arena !== out.arena) throw new Error('siluMul: tensors must share one arena');
        addon.siluMul(this.ctx.handle, gate.arena.handle, gate.offset, up.offset, n, out.offset);
    }
    /** Several linears on one input in one launch (q/k/v, gate/up; qwen.ts:411-413, :464-465). */
    gemmBatch(A, weights, Cs, M) {
        const descs = weights.map((w) => this.linear(w).desc);
        if (!A.pool || Cs.some((c) => c.pool !== A.pool)) throw new Error('gemmBatch: A and every C must come from one ActivationArena');
        const scratch = A.pool.scratchOffset(addon.planBatch(descs, M));
        addon.linearBatch(this.ctx.handle, descs, this.weights.handle, A.arena.handle,
            descs.map(() => A.offset), A.dtype === 'f16' ? QL_DTYPE_F16 : QL_DTYPE_F32, M,
            Cs.map((c) => c.offset), scratch);
    }
    /** fp16 [N,K] copy, bit-identical to the reference's uploaded f16 weight buffer. */
    unpackF16(name, out) {
        const lin = this.linear(name);
        if (out.dtype !== 'f16' || out.length < lin.N * lin.K) throw new Error('unpackF16: output must be an f16 tensor of N*K elements');
        addon.unpack(this.ctx.handle, lin.desc, this.weights.handle, out.arena.handle, out.offset, false);
    }
    /**
     * fp16 [N,K] copies of many weights at once (the loader's whole weight set,
     * qwen-loader.ts:146-162): names[i] into outs[i], same bits as unpackF16, in a few launches.
     */
    unpackAllF16(names, outs) {
        if (names.length !== outs.length) throw new Error('unpackAllF16: one output tensor per weight');
        const descs = names.map((n, i) => {
            const lin = this.linear(n);
            const out = outs[i];
            if (out.dtype !== 'f16' || out.length < lin.N * lin.K) throw new Error('unpackAllF16: output must be an f16 tensor of N*K elements');
            if (out.arena !== outs[0].arena) throw new Error('unpackAllF16: all outputs must share one arena');
            return lin.desc;
        });
        if (descs.length) addon.unpackBatch(this.ctx.handle, descs, this.weights.handle, outs[0].arena.handle, outs.map((o) => o.offset));
    }
    /** fp32 [N,K] = dequantizeGptqInt4 of the stored tensors (computed on the GPU). */
    dequantize(name) {
        const lin = this.linear(name);
        const tmp = this.ctx.arena(lin.N * lin.K * 4);
        try {
            addon.unpack(this.ctx.handle, lin.desc, this.weights.handle, tmp.handle, 0, true);
            return tmp.read(0, new Float32Array(lin.N * lin.K));
        } finally {
            tmp.release();
        }
    }
    release() { this.weights.release(); }
}

// ------------------------------------------------------------------ qwen-loader.ts

const PROJ = [['qW', 'self_attn.q_proj'], ['kW', 'self_attn.k_proj'], ['vW', 'self_attn.v_proj'],
    ['oW', 'self_attn.o_proj'], ['gateW', 'mlp.gate_proj'], ['upW', 'mlp.up_proj'], ['downW', 'mlp.down_proj']];
const BIASED = new Set(['qW', 'kW', 'vW']);

function qwenLinearShapes(c) {
    const C = c.nEmbd, HI = qwenKvDim(c), I = c.intermediate;
    return { qW: [C, C], kW: [C, HI], vW: [C, HI], oW: [C, C], gateW: [C, I], upW: [C, I], downW: [I, C] };
}

const QWEN_LOCAL_DIR = 'models/qwen2.5-0.5b-int4/';   // qwen-loader.ts:27 (public/models layout)

/** A local path or file:// URL -> path (the reference fetches `url`; this host has no network). */
function urlToPath(url) {
    if (/^file:/i.test(url)) return decodeURIComponent(new URL(url).pathname);
    if (/^[a-z][a-z0-9+.-]*:\/\//i.test(url)) throw new Error(`qwen-loader: cannot load ${url}: only a local path or a file:// URL`);
    return url;
}

/** readF16Rows (qwen-loader.ts:70-93): rows [rowStart, rowStart+rowCount) of an F16 tensor as fp32. */
function readF16Rows(file, name, rowStart, rowCount, rowLength) {
    const entry = requireTensor(file, name);
    if (entry.dtype !== 'F16') throw new Error(`qwen-loader: ${name} expected F16, got ${entry.dtype}`);
    if (entry.shape.length !== 2 || entry.shape[0] * rowLength !== entry.shape[0] * entry.shape[1]) {
        throw new Error(`qwen-loader: ${name} shape ${entry.shape} does not match rowLength=${rowLength}`);
    }
    if (rowStart < 0 || rowCount < 0 || rowStart + rowCount > entry.shape[0]) {
        throw new Error(`qwen-loader: rows [${rowStart}, ${rowStart + rowCount}) outside ${name} [${entry.shape}]`);
    }
    const byteStart = file.dataStart + entry.data_offsets[0] + rowStart * rowLength * 2;
    const view = new DataView(file.buffer.buffer, file.buffer.byteOffset + byteStart, rowCount * rowLength * 2);
    const out = new Float32Array(rowCount * rowLength);
    for (let i = 0; i < out.length; i++) out[i] = f16BitsToF32(view.getUint16(i * 2, true));
    return out;
}

/**
 * desc_act=false: g_idx, when present, must be the identity map i / group (qwen-format.ts:125-130).
 * The fused kernels assume it, so an act-order checkpoint is rejected rather than loaded wrong.
 */
function checkGIdx(file, prefix, inFeatures, group) {
    const name = `${prefix}.g_idx`;
    if (!Object.prototype.hasOwnProperty.call(file.header, name)) return;
    expectTensor(file, name, 'I32', [inFeatures]);
    const b = readTensorBytes(file, name);
    const view = new DataView(b.buffer, b.byteOffset, b.byteLength);
    for (let i = 0; i < inFeatures; i++) {
        const g = view.getInt32(i * 4, true);
        if (g !== Math.floor(i / group)) {
            throw new Error(`qwen-loader: ${name}[${i}] = ${g} is not the identity map i/${group} (desc_act checkpoints are not supported)`);
        }
    }
}

/** Adds the stored qzeros nibbles of a linear's real columns into counts[0..15] (qwen-format.ts:112-123). */
function countStoredZeros(qzeros, groups, outFeatures, counts) {
    const nc = Math.ceil(outFeatures / 8);
    const view = new DataView(qzeros.buffer, qzeros.byteOffset, qzeros.byteLength);
    for (let g = 0; g < groups; g++) {
        for (let n = 0; n < outFeatures; n++) {
            const word = view.getUint32((g * nc + (n >> 3)) * 4, true);
            counts[(word >>> (4 * (n & 7))) & 15]++;
        }
    }
    return counts;
}

/**
 * loadQwenWeights (qwen-loader.ts:102-177) for a QuantLinearModel: async, like the reference
 * (`ctx` is unused, as the reference's `_gpu` is; the model holds its context). options (the
 * reference's QwenLoadOptions, qwen-loader.ts:29-38): url (a local path or file:// URL, default
 * QWEN_LOCAL_DIR + 'model.safetensors'), onProgress(done, total, label), keepLayer,
 * keepEmbedRows {start, rows}; and this host's config, groupSize, and path / buffer (a path or an
 * already-read file instead of url). The int4 tensors go to the GPU packed after the shape checks
 * of qwen-format.ts:72-80 and its g_idx identity check; the result (QwenLoadResult, :40-52) adds
 * storedZeros {nibble: count} over every linear (the format probe's stored-zero set, :112-123).
 */
async function loadQwenWeights(ctx, model, options) {
    const opt = options || {};
    const config = opt.config || QWEN25_05B;
    const group = opt.groupSize || 128;
    let raw = opt.buffer;
    if (!raw) {
        const file = opt.path || urlToPath(opt.url !== undefined ? opt.url : `${QWEN_LOCAL_DIR}model.safetensors`);
        raw = await fs.promises.readFile(file);
    }
    const file = parseSafetensors(raw);
    const C = config.nEmbd;
    let tensorCount = 0;
    const emb = requireTensor(file, 'model.embed_tokens.weight');
    if (emb.shape.join(',') !== `${config.vocabSize},${C}`) {
        throw new Error(`qwen-loader: embed_tokens shape [${emb.shape}], expected [${config.vocabSize},${C}]`);
    }
    if (emb.dtype !== 'F16') throw new Error(`qwen-loader: model.embed_tokens.weight expected F16, got ${emb.dtype}`);
    model.uploadF16Bits('embed', readTensorBytes(file, 'model.embed_tokens.weight'), [config.vocabSize, C]);
    tensorCount += 1;
    const embedRows = opt.keepEmbedRows
        ? readF16Rows(file, 'model.embed_tokens.weight', opt.keepEmbedRows.start, opt.keepEmbedRows.rows, C)
        : undefined;
    model.uploadF32('finalNorm', readTensorF32(file, 'model.norm.weight'));
    tensorCount += 1;
    const shapes = qwenLinearShapes(config);
    const zeros = new Array(16).fill(0);
    let kept;
    for (let i = 0; i < config.nLayer; i++) {
        const p = `model.layers.${i}`;
        model.uploadF32(`L${i}.inNorm`, readTensorF32(file, `${p}.input_layernorm.weight`));
        model.uploadF32(`L${i}.postNorm`, readTensorF32(file, `${p}.post_attention_layernorm.weight`));
        tensorCount += 2;
        const layer = {};
        for (const [key, proj] of PROJ) {
            const [K, N] = shapes[key];
            const pre = `${p}.${proj}`;
            const G = Math.ceil(K / group);
            expectTensor(file, `${pre}.qweight`, 'I32', [Math.ceil(K / 8), N]);
            expectTensor(file, `${pre}.qzeros`, 'I32', [G, Math.ceil(N / 8)]);
            expectTensor(file, `${pre}.scales`, 'F16', [G, N]);
            checkGIdx(file, pre, K, group);
            const qzeros = readTensorBytes(file, `${pre}.qzeros`);
            countStoredZeros(qzeros, G, N, zeros);
            const bias = BIASED.has(key) ? readTensorF32(file, `${pre}.bias`) : null;
            model.uploadGptqLinear(`L${i}.${key}`, {
                qweight: readTensorBytes(file, `${pre}.qweight`), qzeros,
                scalesF16: readTensorBytes(file, `${pre}.scales`), inFeatures: K, outFeatures: N,
                groupSize: group, bias,
            });
            tensorCount += bias ? 2 : 1;
            if (opt.keepLayer === i) layer[key] = model.dequantize(`L${i}.${key}`);
        }
        if (opt.keepLayer === i) kept = layer;
        if (opt.onProgress) opt.onProgress(i + 1, config.nLayer, `layer ${i + 1}/${config.nLayer}`);
    }
    const storedZeros = {};
    zeros.forEach((c, v) => { if (c) storedZeros[v] = c; });
    return { gpuBytes: model.weightBytes, tensorCount, fileBytes: raw.byteLength, layer: kept, embedRows, storedZeros };
}

/**
 * Per-layer fp32 K and V caches [blockSize, nKvHead * headDim] and the decode attention over them:
 * QwenGpt's kCache/vCache (qwen.ts:140-141, :200-205), kv_store (:427-428), attention_gqa_cache (:429-440).
 */
class KvCache {
    constructor(ctx, config) {
        this.ctx = ctx;
        this.config = config;
        this.D = qwenHeadDim(config);
        this.rowLen = qwenKvDim(config);
        this.region = Math.ceil(config.blockSize * this.rowLen * 4 / 256) * 256;
        this.arena = ctx.arena(2 * config.nLayer * this.region);
    }
    offsets(layer) {
        if (layer < 0 || layer >= this.config.nLayer) throw new Error(`layer ${layer} out of range`);
        return [2 * layer * this.region, (2 * layer + 1) * this.region];
    }
    store(layer, k, v, rows, pos0) {
        const [ko, vo] = this.offsets(layer);
        if (k.arena !== v.arena) throw new Error('store: k and v must share one arena');
        addon.kvStore(this.ctx.handle, k.arena.handle, k.offset, this.arena.handle, ko, this.config.blockSize, rows, this.rowLen, pos0);
        addon.kvStore(this.ctx.handle, v.arena.handle, v.offset, this.arena.handle, vo, this.config.blockSize, rows, this.rowLen, pos0);
    }
    attend(layer, q, out, M, pastLen) {
        const c = this.config;
        if (q.arena !== out.arena) throw new Error('attend: q and out must share one arena');
        const [ko, vo] = this.offsets(layer);
        addon.attention(this.ctx.handle, q.arena.handle, q.offset, this.arena.handle, ko, vo, c.blockSize, M,
            c.nHead, c.nKvHead, this.D, pastLen, out.offset);
    }
    release() { this.arena.release(); }
}

module.exports = {
    addon, ADDON_PATH, QL_DTYPE_F32, QL_DTYPE_F16, QWEN25_05B, qwenHeadDim, qwenKvDim, Seq,
    dtypeByteSize, parseSafetensorsHeader, parseSafetensors, tensorCount, requireTensor,
    expectTensor, f16BitsToF32, readTensorBytes, readTensorF32, ArenaLayout, Arena, Context,
    makeDesc, dequantizeGptqInt4, Tensor, ActivationArena, QuantLinearModel,
    qwenLinearShapes, loadQwenWeights, KvCache, QWEN_LOCAL_DIR, urlToPath, readF16Rows, checkGIdx,
    countStoredZeros,
};
