/**
 * L6 · model hyper-parameters.  Same fields, defaults and derived dimensions
 * as forge-llm's Config (src/L6/transformer.js:29-53), including the GQA
 * divisibility check.
 */
function pick(o, k, d) { return o[k] === undefined || o[k] === null ? d : o[k]; }

export class Config {
  constructor(o = {}) {
    this.dim = pick(o, "dim", 288);
    this.hidden = pick(o, "hidden", 768);
    this.nLayers = pick(o, "nLayers", 6);
    this.nHeads = pick(o, "nHeads", 6);
    this.nKvHeads = pick(o, "nKvHeads", 6);
    this.vocabSize = pick(o, "vocabSize", 32000);
    this.maxSeq = pick(o, "maxSeq", 1024);
    this.normEps = pick(o, "normEps", 1e-5);
    this.ropeTheta = pick(o, "ropeTheta", 10000);
    this.bosId = pick(o, "bosId", 1);
    this.eosId = pick(o, "eosId", 2);
    this._derive();
  }
  _derive() {
    if (this.nHeads % this.nKvHeads !== 0) {
      throw new Error(`GQA needs nHeads (${this.nHeads}) divisible by nKvHeads (${this.nKvHeads})`);
    }
    this.dHead = Math.floor(this.dim / this.nHeads);
    this.kvDim = this.nKvHeads * this.dHead;
    this.qkvOut = (this.nHeads + 2 * this.nKvHeads) * this.dHead;
    this.groupSize = this.nHeads / this.nKvHeads;
  }
}
