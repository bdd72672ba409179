CacheDType = str
