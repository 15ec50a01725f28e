/* placeholder until the obs/reward restatement lands */
