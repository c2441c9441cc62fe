// Types of the Node host for libqlinear (index.js), for the reference's TypeScript code.

export interface QwenConfig {
    vocabSize: number; blockSize: number; nLayer: number; nHead: number; nKvHead: number;
    nEmbd: number; intermediate: number; rmsEps?: number; ropeTheta?: number;
}
export const QWEN25_05B: Readonly<QwenConfig>;
export function qwenHeadDim(c: QwenConfig): number;
export function qwenKvDim(c: QwenConfig): number;

export type SafetensorDtype = 'F64' | 'F32' | 'F16' | 'BF16' | 'I64' | 'I32' | 'I16' | 'I8' | 'U8' | 'BOOL';
export interface SafetensorEntry { dtype: SafetensorDtype; shape: number[]; data_offsets: [number, number]; }
export interface SafetensorFile { buffer: Uint8Array; dataStart: number; header: Record<string, SafetensorEntry>; }
export function dtypeByteSize(dtype: SafetensorDtype): number;
export function parseSafetensorsHeader(headerBytes: Uint8Array): Record<string, SafetensorEntry>;
export function parseSafetensors(buffer: ArrayBuffer | Uint8Array): SafetensorFile;
export function tensorCount(entry: SafetensorEntry): number;
export function requireTensor(file: SafetensorFile, name: string): SafetensorEntry;
export function expectTensor(file: SafetensorFile, name: string, dtype: SafetensorDtype, shape: readonly number[]): SafetensorEntry;
export function f16BitsToF32(bits: number): number;
export function readTensorBytes(file: SafetensorFile, name: string): Uint8Array;
export function readTensorF32(file: SafetensorFile, name: string): Float32Array;

/** Error thrown by the library: `code` is 'QL_E_*'. */
export interface QlError extends Error { code: string; }

export interface GptqDesc {
    qweightOff: number; qzerosOff: number | null; scalesOff: number; biasOff: number | null;
    K: number; N: number; group: number; bits: number;
}
export function makeDesc(qweightOff: number, qzerosOff: number | null, scalesOff: number, K: number,
                         N: number, group?: number, biasOff?: number | null, bits?: number): GptqDesc;

export class ArenaLayout { used: number; take(nbytes: number, align?: number): number; }
export class Arena {
    readonly size: number;
    write(off: number, data: ArrayBufferView): void;
    read<T extends ArrayBufferView>(off: number, into: T): T;
    release(): void;
}
export interface SeqInfo {
    linears: number; passes: number; tiles: number; reduces: number; grid: number;
    maxSplit: number; ldsBytes: number; deviceBytes: number;
    /** block-groups (64 columns x one group) in total and on the busiest workgroup */
    totalUnits: number; busiestUnits: number;
    /** 0: dependency-ordered tiles, 1: column strips; split: waves per 64-column block of a strip */
    kernel: number; split: number;
}
/** A forward's decode linears (M <= 16) as one persistent launch; linear i reads linear j's
 *  output when xOffs[i] === yOffs[j]. */
export class Seq {
    readonly info: SeqInfo;
    run(): void;
    status(): void;
    destroy(): void;
}
/** Elementwise work folded into one linear of a fused sequence (ql_seq_fuse). */
export interface SeqFuse {
    normWOff?: number | null; normEps?: number; x2Off?: number | null; resOff?: number | null;
}
export class Context {
    constructor(device?: number);
    seq(descs: GptqDesc[], weights: Arena, act: Arena, xOffs: number[], xDtype: number, M: number,
        yOffs: number[], fuse?: (SeqFuse | null)[]): Seq;
    info(): { name: string; cuCount: number; hbmBytes: number };
    arena(bytes: number): Arena;
    sync(): void;
    timerStart(): void;
    timerStop(): number;
    destroy(): void;
}

export interface GptqInt4Params {
    qweight: Uint8Array; qzeros?: Uint8Array | null; scales: Float32Array;
    inFeatures: number; outFeatures: number; groupSize?: number; bits?: number;
}
/** quant.ts dequantizeGptqInt4, computed on the GPU: fp32 [outFeatures, inFeatures], for any f32 scales. */
export function dequantizeGptqInt4(params: GptqInt4Params, ctx?: Context): Float32Array;

export class Tensor {
    readonly arena: Arena; readonly offset: number; readonly length: number;
    readonly shape: number[]; readonly dtype: 'f32' | 'f16' | 'u32';
    read(): Float32Array | Uint16Array | Uint32Array;
    write(data: ArrayBufferView): void;
}
export class ActivationArena {
    constructor(ctx: Context, bytes: number);
    alloc(shape: number[], dtype?: 'f32' | 'f16' | 'u32'): Tensor;
    scratchOffset(nbytes: number): number;
    reset(): void;
    release(): void;
}
export interface GptqLinearUpload {
    qweight: Uint8Array; qzeros?: Uint8Array | null; scalesF16: Uint8Array | Uint16Array;
    inFeatures: number; outFeatures: number; groupSize?: number; bias?: Float32Array | null;
}
export class QuantLinearModel {
    constructor(ctx: Context, weightCapacity: number);
    readonly weightBytes: number;
    uploadGptqLinear(name: string, p: GptqLinearUpload): void;
    uploadF32(name: string, data: ArrayLike<number>): void;
    uploadF16Bits(name: string, bytes: ArrayBufferView, shape: number[]): void;
    /** QwenGpt.gemm: C[M,N] = A[M,K] @ W^T (+ bias). */
    gemm(A: Tensor, weight: string, C: Tensor, bias: string | null, M: number, N: number, K: number): void;
    gemmBatch(A: Tensor, weights: string[], Cs: Tensor[], M: number): void;
    /** out[M, C] = the fp16 table's rows tokens[0..M) as f32 (ql_embed_f16); ids >= vocab give zeros. */
    embed(tokens: Tensor, out: Tensor, M: number, weight?: string): void;
    /** y = rmsnorm(x (+ residual)) * weight, the sum stored in sumOut (one launch: ql_add_rmsnorm). */
    rmsnorm(x: Tensor, weight: string, y: Tensor, M: number, C: number, eps: number,
            residual?: Tensor | null, sumOut?: Tensor | null): void;
    /** out = silu(gate) * up (ql_silu_mul). */
    siluMul(gate: Tensor, up: Tensor, out: Tensor, n: number): void;
    unpackF16(name: string, out: Tensor): void;
    /** fp16 [N,K] copies of many weights in a few launches (ql_unpack_f16_batch). */
    unpackAllF16(names: string[], outs: Tensor[]): void;
    dequantize(name: string): Float32Array;
    release(): void;
}

/** Per-layer fp32 K/V caches and decode attention (qwen.ts:200-205, :427-440). */
export class KvCache {
    constructor(ctx: Context, config: QwenConfig);
    readonly D: number;
    readonly rowLen: number;
    store(layer: number, k: Tensor, v: Tensor, rows: number, pos0: number): void;
    attend(layer: number, q: Tensor, out: Tensor, M: number, pastLen: number): void;
    release(): void;
}

/** qwen-loader.ts:29-38, plus this host's config / groupSize and path / buffer alternatives to url. */
export interface QwenLoadOptions {
    /** a local path or file:// URL; default QWEN_LOCAL_DIR + 'model.safetensors' */
    url?: string;
    onProgress?: (done: number, total: number, label: string) => void;
    keepLayer?: number;
    keepEmbedRows?: { start: number; rows: number };
    path?: string; buffer?: ArrayBuffer | Uint8Array; config?: QwenConfig; groupSize?: number;
}
/** qwen-loader.ts:40-52, plus storedZeros: {nibble: count} of the stored qzeros (qwen-format.ts:112-123). */
export interface QwenLoadResult {
    gpuBytes: number; tensorCount: number; fileBytes: number;
    layer?: Record<'qW' | 'kW' | 'vW' | 'oW' | 'gateW' | 'upW' | 'downW', Float32Array>;
    embedRows?: Float32Array;
    storedZeros: Record<number, number>;
}
export const QWEN_LOCAL_DIR: string;
export function qwenLinearShapes(c: QwenConfig): Record<string, [number, number]>;
/** Rejects (throws asynchronously) on a malformed file, wrong shapes or a non-identity g_idx. */
export function loadQwenWeights(ctx: Context | null, model: QuantLinearModel, options?: QwenLoadOptions): Promise<QwenLoadResult>;
export function urlToPath(url: string): string;
export function readF16Rows(file: SafetensorFile, name: string, rowStart: number, rowCount: number, rowLength: number): Float32Array;
export function checkGIdx(file: SafetensorFile, prefix: string, inFeatures: number, group: number): void;
export function countStoredZeros(qzeros: Uint8Array, groups: number, outFeatures: number, counts: number[]): number[];
