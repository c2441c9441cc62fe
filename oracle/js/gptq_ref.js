#!/usr/bin/env node
/*
 * CPU baseline for the GPTQ int4 linear path — TEST/BENCH INFRASTRUCTURE ONLY.
 *
 * A Node-runnable (ES2019, runs on Node 12) restatement of the reference's CPU path
 * (intplusplus/webllm, TypeScript), used by bench.py's cpu_baseline leg and never by the product:
 *   f16BitsToF32        src/weights/safetensors.ts:144-152 (scales F16 -> f32, :180-182)
 *   dequantizeGptqInt4  src/weights/quant.ts:42-118 (DataView word reads, stored zero + 1)
 *   gemmNTRef           src/reference/qwen-ref.ts:126-145 (JS-number accumulator, ascending k)
 *
 *   f32ToF16Bits        src/gpu/buffer.ts:57-104 (RNE to binary16; the load-time fp16 arena)
 *
 * Usage: node gptq_ref.js <dir> [min_seconds]
 *   <dir>/meta.json: {"linears":[{"K":..,"N":..,"group":..,"qweight":"f","qzeros":"f"|null,
 *                     "scales":"f","x":"f","M":..}],
 *                     "plan": {"fused_reps": R, "f16_reps": R}}   (plan optional)
 *   raw little-endian files: qweight u32, qzeros u32, scales f16 bits, x f32 [M,K].
 * Prints one JSON line of timings (performance.now, single thread) and writes the matvec outputs
 * to <dir>/y_<i>.f32 for comparison with the GPU:
 *   dequant_ms      all linears dequantized once (the reference's load step)
 *   matvec_ms       variant (i): the matvecs over the dequantized weights, mean over the reps of
 *                   min_seconds of work; matvec_median_ms their median
 *   fused_ms        variant (ii), plan.fused_reps > 0: dequant + matvec per call, median
 *   f16_ms          plan.f16_reps > 0: dequant + f32ToF16Bits of every weight (the fp16 unpack of
 *                   config 5), median
 */
'use strict';
const fs = require('fs');
const path = require('path');
const { performance } = require('perf_hooks');
const os = require('os');

function f16BitsToF32(bits) {
  const sign = (bits & 0x8000) !== 0 ? -1 : 1;
  const exp = (bits >>> 10) & 0x1f;
  const mant = bits & 0x03ff;
  if (exp === 0) return sign * mant * Math.pow(2, -24);
  if (exp === 31) return mant === 0 ? sign * Infinity : NaN;
  return sign * (1 + mant / 1024) * Math.pow(2, exp - 15);
}

function dequantizeGptqInt4(params) {
  const groupSize = params.groupSize === undefined ? 128 : params.groupSize;
  const bits = params.bits === undefined ? 4 : params.bits;
  if (bits !== 4) throw new Error('GPTQ: bits must be 4, got ' + bits);
  if (groupSize <= 0) throw new Error('GPTQ: groupSize must be positive');
  if (params.inFeatures <= 0 || params.outFeatures <= 0) throw new Error('GPTQ: in/out must be positive');
  const inF = params.inFeatures;
  const outF = params.outFeatures;
  const packFactor = 32 / bits;
  const mask = (1 << bits) - 1;
  const packRows = Math.ceil(inF / packFactor);
  const packCols = Math.ceil(outF / packFactor);
  const groups = Math.ceil(inF / groupSize);
  if (params.qweight.byteLength < packRows * outF * 4) throw new Error('GPTQ: qweight too short');
  if (params.scales.length < groups * outF) throw new Error('GPTQ: scales too short');
  const qwView = new DataView(params.qweight.buffer, params.qweight.byteOffset, params.qweight.byteLength);
  const qzView = params.qzeros
    ? new DataView(params.qzeros.buffer, params.qzeros.byteOffset, params.qzeros.byteLength) : null;
  if (qzView && qzView.byteLength < groups * packCols * 4) throw new Error('GPTQ: qzeros too short');
  const symmetricZero = 1 << (bits - 1);
  if (groupSize % packFactor !== 0) throw new Error('GPTQ: groupSize must be a multiple of 8');
  const out = new Float32Array(outF * inF);
  for (let packRow = 0; packRow < packRows; packRow++) {
    const rowBase = packRow * packFactor;
    const g = (rowBase / groupSize) | 0;
    const qwRowBase = packRow * outF;
    for (let o = 0; o < outF; o++) {
      const word = qwView.getUint32((qwRowBase + o) * 4, true);
      const scale = params.scales[g * outF + o];
      let zero;
      if (qzView) {
        const zWord = qzView.getUint32((g * packCols + ((o / packFactor) | 0)) * 4, true);
        zero = ((zWord >>> (bits * (o % packFactor))) & mask) + 1;
      } else {
        zero = symmetricZero;
      }
      const outIndex = o * inF;
      for (let k = 0; k < packFactor; k++) {
        const i = rowBase + k;
        if (i >= inF) break;
        const q = (word >>> (bits * k)) & mask;
        out[outIndex + i] = (q - zero) * scale;
      }
    }
  }
  return out;
}

// IEEE binary16 bits of an f32 value, round to nearest even (any NaN -> 0x7e00, overflow -> inf,
// |value| < 2^-24 -> signed zero, as buffer.ts:73 does, where IEEE RNE would give 0x0001 above
// 2^-25).
const F16_SCRATCH_F = new Float32Array(1);
const F16_SCRATCH_U = new Uint32Array(F16_SCRATCH_F.buffer);
function f32ToF16Bits(value) {
  F16_SCRATCH_F[0] = value;
  const u = F16_SCRATCH_U[0];
  const sign = (u >>> 16) & 0x8000;
  const e8 = (u >>> 23) & 0xff;
  const m23 = u & 0x7fffff;
  if (e8 === 0xff) return m23 !== 0 ? 0x7e00 : sign | 0x7c00;   // every NaN -> 0x7e00
  const e = e8 - 127;
  if (e > 15) return sign | 0x7c00;
  if (e < -24) return sign;
  let m, drop;
  if (e < -14) {             // subnormal half: keep 10 - (-14 - e) bits of the 24-bit significand
    m = m23 | 0x800000;
    drop = -1 - e;           // 14..23
  } else {
    m = m23;
    drop = 13;
  }
  let h = m >>> drop;
  const rest = m - (h << drop);
  const half = 1 << (drop - 1);
  if (rest > half || (rest === half && (h & 1) === 1)) h++;
  if (e < -14) return sign | h;             // a carry into bit 10 is the smallest normal
  return sign | ((((e + 15) << 10) + h) & 0x7fff);   // a mantissa carry steps the exponent
}

function gemmNTRef(A, W, M, N, K, bias) {
  const C = new Float32Array(M * N);
  for (let m = 0; m < M; m++) {
    for (let n = 0; n < N; n++) {
      let acc = 0;
      const aBase = m * K;
      const wBase = n * K;
      for (let k = 0; k < K; k++) acc += A[aBase + k] * W[wBase + k];
      C[m * N + n] = bias ? acc + bias[n] : acc;
    }
  }
  return C;
}

function readRaw(dir, name) {
  const buf = fs.readFileSync(path.join(dir, name));
  return new Uint8Array(buf.buffer, buf.byteOffset, buf.byteLength);
}

function main() {
  const dir = process.argv[2];
  const minSeconds = process.argv.length > 3 ? Number(process.argv[3]) : 5;
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
  const linears = meta.linears.map((d) => {
    const qweight = readRaw(dir, d.qweight);
    const qzeros = d.qzeros ? readRaw(dir, d.qzeros) : null;
    const sBytes = readRaw(dir, d.scales);
    const sView = new DataView(sBytes.buffer, sBytes.byteOffset, sBytes.byteLength);
    const xBytes = readRaw(dir, d.x);
    const x = new Float32Array(xBytes.buffer.slice(xBytes.byteOffset, xBytes.byteOffset + xBytes.byteLength));
    return { d, qweight, qzeros, sView, x };
  });

  const plan = meta.plan || {};
  // load time: scales F16 -> f32 and dequant (the reference does this once per load)
  const dequant = (L) => {
    const G = Math.ceil(L.d.K / L.d.group);
    const scales = new Float32Array(G * L.d.N);
    for (let i = 0; i < scales.length; i++) scales[i] = f16BitsToF32(L.sView.getUint16(i * 2, true));
    return dequantizeGptqInt4({ qweight: L.qweight, qzeros: L.qzeros, scales,
      inFeatures: L.d.K, outFeatures: L.d.N, groupSize: L.d.group });
  };
  const t0 = performance.now();
  const weights = linears.map(dequant);
  const dequantMs = performance.now() - t0;

  // variant (i), per step: the matvecs (repeated until min_seconds of work)
  const times = [];
  const t1 = performance.now();
  let outs = null;
  do {
    const ts = performance.now();
    outs = linears.map((L, i) => gemmNTRef(L.x, weights[i], L.d.M, L.d.N, L.d.K, null));
    times.push(performance.now() - ts);
  } while (performance.now() - t1 < minSeconds * 1000 || times.length < 3);
  const reps = times.length;
  const matvecMs = (performance.now() - t1) / reps;
  outs.forEach((y, i) => fs.writeFileSync(path.join(dir, 'y_' + i + '.f32'), Buffer.from(y.buffer)));
  weights.length = 0;
  const median = (v) => { const s = v.slice().sort((a, b) => a - b); return s[(s.length - 1) >> 1]; };

  // variant (ii): dequant + matvec per call
  let fusedMs = null;
  if (plan.fused_reps > 0) {
    const ft = [];
    for (let r = 0; r < plan.fused_reps; r++) {
      const ts = performance.now();
      linears.forEach((L) => gemmNTRef(L.x, dequant(L), L.d.M, L.d.N, L.d.K, null));
      ft.push(performance.now() - ts);
    }
    fusedMs = median(ft);
  }
  // the fp16 unpack: dequant + RNE binary16 of every weight ([N, K] layout)
  let f16Ms = null;
  if (plan.f16_reps > 0) {
    const ht = [];
    for (let r = 0; r < plan.f16_reps; r++) {
      const ts = performance.now();
      linears.forEach((L) => {
        const w = dequant(L);
        const h = new Uint16Array(w.length);
        for (let i = 0; i < w.length; i++) h[i] = f32ToF16Bits(w[i]);
      });
      ht.push(performance.now() - ts);
    }
    f16Ms = median(ht);
  }
  const macs = linears.reduce((a, L) => a + L.d.M * L.d.N * L.d.K, 0);
  process.stdout.write(JSON.stringify({
    node: process.version, cpu: os.cpus()[0].model, cpus: os.cpus().length, threads: 1,
    linears: linears.length, macs, dequant_ms: dequantMs, matvec_ms: matvecMs,
    matvec_median_ms: median(times), reps, fused_ms: fusedMs, f16_ms: f16Ms,
  }) + '\n');
}

if (process.argv[2] === '--f16-selftest') {
  // f32ToF16Bits over given f32 bit patterns (stdin: JSON array of u32), for the tests
  const bitsIn = JSON.parse(fs.readFileSync(0, 'utf8'));
  const f = new Float32Array(1);
  const u = new Uint32Array(f.buffer);
  process.stdout.write(JSON.stringify(bitsIn.map((b) => { u[0] = b >>> 0; return f32ToF16Bits(f[0]); })) + '\n');
} else {
  main();
}

